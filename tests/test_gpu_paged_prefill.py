"""Multi-query attention over the paged cache (code step and prompt chunks) vs the fp64 oracle
(tolerance: max-abs <= 2e-2 for bf16 outputs and LSE)."""
import numpy as np
import pytest
import torch

from oracle import decode as od

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _setup(n_rows, n_pages, seed):
    rng = np.random.default_rng(seed)
    need = [-(-n // 16) for n in n_rows]
    perm = rng.permutation(np.arange(1, n_pages))
    W = max(need)
    tables = np.zeros((len(n_rows), W), np.int32)
    at = 0
    for r, n in enumerate(need):
        tables[r, :n] = perm[at: at + n]
        at += n
    g = torch.Generator().manual_seed(seed)
    cache = torch.randn((n_pages, 2, 16, 8, 128), generator=g).to(torch.bfloat16)
    return cache, tables


def _oracle(q_rows, cache, table, kv_start, limit, causal, excluded=None):
    """fp64 attention of query rows q_rows [n, 32, 128] at positions kv_start + i over physical keys < limit (minus
    the excluded range)."""
    out = np.zeros((len(q_rows), 32, 128))
    lse = np.zeros((len(q_rows), 32))
    k, v = od.paged_rows(cache, table, limit)
    for i in range(len(q_rows)):
        n = min(limit, kv_start + i + 1) if causal else limit
        keep = np.arange(n)
        if excluded is not None:
            keep = keep[(keep < excluded[0]) | (keep >= excluded[1])]
        out[i], lse[i] = od.decode_fp64(q_rows[i], k[keep], v[keep], 128 ** -0.5)
    return out, lse


def _run(cache_bf, tables, q, q_start, kv_start, kv_limit, causal, split=None, excluded=None):
    from abridgekv_amd import ops
    dev = torch.device("cuda")
    lse = torch.empty((q.shape[0], 32), dtype=torch.float32, device=dev)
    out, _ = ops.paged_prefill_attention(q.to(dev), cache_bf.to(dev), torch.from_numpy(tables).to(dev), q_start,
                                         kv_start, kv_limit, causal, lse=lse, split=split, excluded=excluded)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), lse.cpu().numpy()


@pytest.mark.parametrize("split", [None, 1, 3, 7])
def test_code_step_limits_per_group_quota(split):
    """K=256 code queries per request at physical positions [R, R+256), visible keys < R + q (own slots >= q hidden);
    with the keys split over several workgroups and merged, or not."""
    resident = [700, 1301, 45]
    quotas = [64, 256, 128]
    cache, tables = _setup([r + 256 for r in resident], 400, 0)
    g = torch.Generator().manual_seed(1)
    q = torch.randn((3 * 256, 32, 128), generator=g).to(torch.bfloat16)
    q_start = [0, 256, 512, 768]
    kv_limit = [r + qq for r, qq in zip(resident, quotas)]
    out, lse = _run(cache, tables, q, q_start, resident, kv_limit, causal=False, split=split)
    cf = cache.float().numpy()
    for r in range(3):
        ro, rl = _oracle(q[q_start[r]: q_start[r + 1]].float().numpy(), cf, tables[r], resident[r], kv_limit[r],
                         causal=False)
        assert np.abs(out[q_start[r]: q_start[r + 1]] - ro).max() <= TOL
        assert np.abs(lse[q_start[r]: q_start[r + 1]] - rl).max() <= TOL


@pytest.mark.parametrize("split", [None, 1, 5])
def test_code_step_static_tail_excluded(split):
    """Code steps whose block's last T content rows (just before the code rows) are hidden from the codes: T = 64
    aligned to a tile, T = 37 across a tile boundary, T = 200 spanning whole tiles (one of them entirely hidden), and
    a request without a range in the same launch."""
    resident = [700, 1301, 460, 900]
    quotas = [64, 256, 128, 32]
    tails = [64, 37, 200, None]
    cache, tables = _setup([r + 256 for r in resident], 400, 7)
    g = torch.Generator().manual_seed(8)
    q = torch.randn((4 * 256, 32, 128), generator=g).to(torch.bfloat16)
    q_start = [0, 256, 512, 768, 1024]
    kv_limit = [r + qq for r, qq in zip(resident, quotas)]
    excluded = [None if t is None else (r - t, r) for r, t in zip(resident, tails)]
    out, lse = _run(cache, tables, q, q_start, resident, kv_limit, causal=False, split=split, excluded=excluded)
    cf = cache.float().numpy()
    for r in range(4):
        ro, rl = _oracle(q[q_start[r]: q_start[r + 1]].float().numpy(), cf, tables[r], resident[r], kv_limit[r],
                         causal=False, excluded=excluded[r])
        assert np.abs(out[q_start[r]: q_start[r + 1]] - ro).max() <= TOL, r
        assert np.abs(lse[q_start[r]: q_start[r + 1]] - rl).max() <= TOL, r


def test_causal_prompt_chunks_ragged():
    """Causal chunks with prior context: 300 rows after 500 resident, a single-query request, a 64-row chunk at 0."""
    nq = [300, 1, 64, 77]
    kv_start = [500, 999, 0, 130]
    lens = [s + n for s, n in zip(kv_start, nq)]
    cache, tables = _setup(lens, 300, 2)
    g = torch.Generator().manual_seed(3)
    q_start = np.concatenate([[0], np.cumsum(nq)]).tolist()
    q = torch.randn((q_start[-1], 32, 128), generator=g).to(torch.bfloat16)
    out, lse = _run(cache, tables, q, q_start, kv_start, lens, causal=True, split=4)
    cf = cache.float().numpy()
    for r in range(len(nq)):
        qr = q[q_start[r]: q_start[r + 1]].float().numpy()
        ro = np.zeros((nq[r], 32, 128))
        rl = np.zeros((nq[r], 32))
        k, v = od.paged_rows(cf, tables[r], lens[r])
        for i in range(nq[r]):
            ro[i], rl[i] = od.decode_fp64(qr[i], k[: kv_start[r] + i + 1], v[: kv_start[r] + i + 1], 128 ** -0.5)
        assert np.abs(out[q_start[r]: q_start[r + 1]] - ro).max() <= TOL
        assert np.abs(lse[q_start[r]: q_start[r + 1]] - rl).max() <= TOL


def test_rejects_limits_past_the_table():
    from abridgekv_amd import ops
    dev = torch.device("cuda")
    cache = torch.zeros((4, 2, 16, 8, 128), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.paged_prefill_attention(torch.zeros((2, 32, 128), dtype=torch.bfloat16, device=dev), cache,
                                    torch.zeros((1, 2), dtype=torch.int32, device=dev), [0, 2], [0], [33], True)


def test_mixed_code_and_prompt_chunk_batch():
    """One launch mixing a non-causal code step (limit = code start + quota) with causal prompt chunks."""
    nq = [256, 130, 1]
    kv_start = [640, 0, 377]
    limits = [640 + 128, 130, 378]
    causal = [False, True, True]
    cache, tables = _setup([max(s + n, l) for s, n, l in zip(kv_start, nq, limits)], 200, 4)
    g = torch.Generator().manual_seed(5)
    q_start = np.concatenate([[0], np.cumsum(nq)]).tolist()
    q = torch.randn((q_start[-1], 32, 128), generator=g).to(torch.bfloat16)
    out, lse = _run(cache, tables, q, q_start, kv_start, limits, causal)
    cf = cache.float().numpy()
    for r in range(len(nq)):
        ro, rl = _oracle(q[q_start[r]: q_start[r + 1]].float().numpy(), cf, tables[r], kv_start[r], limits[r],
                         causal[r])
        assert np.abs(out[q_start[r]: q_start[r + 1]] - ro).max() <= TOL
        assert np.abs(lse[q_start[r]: q_start[r + 1]] - rl).max() <= TOL


def test_rows_past_the_covered_queries_are_untouched_with_key_splits():
    """q_start[-1] < T: the split merge writes only the rows the requests cover; the rest of out keeps its values."""
    from abridgekv_amd import ops
    resident = [900, 1500]
    cache, tables = _setup([r + 64 for r in resident], 300, 5)
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(6)
    T = 200
    q = torch.randn((T, 32, 128), generator=g).to(torch.bfloat16).to(dev)
    out = torch.full((T, 32, 128), 7.0, dtype=torch.bfloat16, device=dev)
    q_start = [0, 64, 128]
    kv_limit = [r + 32 for r in resident]
    ops.paged_prefill_attention(q, cache.to(dev), torch.from_numpy(tables).to(dev), q_start, resident, kv_limit,
                                False, out=out, split=3)
    torch.cuda.synchronize()
    assert bool((out[128:] == 7.0).all())
    cf = cache.float().numpy()
    for r in range(2):
        ro, _ = _oracle(q[q_start[r]: q_start[r + 1]].float().cpu().numpy(), cf, tables[r], resident[r], kv_limit[r],
                        causal=False)
        assert np.abs(out[q_start[r]: q_start[r + 1]].float().cpu().numpy() - ro).max() <= TOL
