"""fp32 mode of the attention paths vs the float64 oracle (tolerance: max-abs <= 1e-5 for outputs and LSE)."""
import numpy as np
import pytest
import torch

from oracle import decode as od
from oracle import masks as om
from oracle import prefill as op

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _paged(lens, num_pages, seed):
    rng = np.random.default_rng(seed)
    need = [-(-n // 16) for n in lens]
    perm = rng.permutation(np.arange(1, num_pages))
    tables = np.zeros((len(lens), max(max(need), 1)), np.int32)
    at = 0
    for r, n in enumerate(need):
        tables[r, :n] = perm[at: at + n]
        at += n
    g = torch.Generator().manual_seed(seed)
    cache = torch.randn((num_pages, 2, 16, 8, 128), generator=g, dtype=torch.float32)
    return cache, tables


def test_decode_f32_matches_fp64():
    from abridgekv_amd import ops
    lens = [1, 17, 300, 1068, 2999, 0]
    cache, tables = _paged(lens, 600, 0)
    g = torch.Generator().manual_seed(1)
    q = torch.randn((len(lens), 32, 128), generator=g, dtype=torch.float32)
    dev = torch.device("cuda")
    lse = torch.empty((len(lens), 32), dtype=torch.float32, device=dev)
    out, _ = ops.decode_attention(q.to(dev), cache.to(dev), torch.from_numpy(tables).to(dev),
                                  torch.tensor(lens, dtype=torch.int32, device=dev), 128 ** -0.5, lse=lse)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    ref_o, ref_l = od.decode_paged_fp64(q.numpy(), cache.numpy(), tables, lens, 128 ** -0.5)
    got_o, got_l = out.cpu().numpy(), lse.cpu().numpy()
    assert np.abs(got_o - ref_o).max() <= TOL
    live = np.asarray(lens) > 0
    assert np.abs(got_l[live] - ref_l[live]).max() <= TOL
    assert np.all(np.isneginf(got_l[~live])) and np.all(got_o[~live] == 0)


@pytest.mark.parametrize("tail", [0, 40])
def test_paged_multi_query_f32_code_step_and_chunks(tail):
    """fp32 code step (key limit code start + quota; with a static tail, the block's last rows before the codes
    excluded: the reference's mask with its excluded range, compresslm_masks.py:206-213) and causal chunks."""
    from abridgekv_amd import ops
    quota, K = 64, 128
    reqs = [(K, 500 + K, (500, 500 + K)), (90, 90 + 200, None), (1, 777, None)]
    excluded = [(500 - tail, 500) if tail and span else None for _, _, span in reqs]
    cache, tables = _paged([sl for _, sl, _ in reqs], 300, 2)
    qsl = np.concatenate([[0], np.cumsum([r[0] for r in reqs])])
    g = torch.Generator().manual_seed(3)
    q = torch.randn((int(qsl[-1]), 32, 128), generator=g, dtype=torch.float32)
    sls = [r[1] for r in reqs]
    kv_start = [sl - ql for ql, sl, _ in reqs]
    limits = [sl if span is None else span[0] + quota for _, sl, span in reqs]
    causal = [span is None for _, _, span in reqs]
    dev = torch.device("cuda")
    lse = torch.empty((int(qsl[-1]), 32), dtype=torch.float32, device=dev)
    out, _ = ops.paged_prefill_attention(q.to(dev), cache.to(dev), torch.from_numpy(tables).to(dev), qsl, kv_start,
                                         limits, causal, lse=lse, excluded=excluded if tail else None)
    torch.cuda.synchronize()
    got_o, got_l = out.cpu().numpy(), lse.cpu().numpy()
    cf = cache.numpy()
    for r, (ql, sl, span) in enumerate(reqs):
        m = om.request_mask(ql, sl, [span] if span else [], excluded[r], quota, K, causal=span is None)
        ro, rl = om.masked_paged_attention_fp64(q[qsl[r]: qsl[r + 1]].numpy(), cf, tables[r], sl, m, 128 ** -0.5)
        assert np.abs(got_o[qsl[r]: qsl[r + 1]] - ro).max() <= TOL, f"request {r}"
        assert np.abs(got_l[qsl[r]: qsl[r + 1]] - rl).max() <= TOL, f"request {r}"


@pytest.mark.parametrize("prompt_len,quota,tail,policy", [(None, None, 0, "static"), ([40, 150], None, 0, "static"),
                                                           ([0, 70], "mixed", 0, "static"),
                                                           ([40, 0], "mixed", 12, "static"),
                                                           ([40, 0], "mixed", 12, "rolling"),
                                                           ([70, 0], "mixed", 20, "sticky"),
                                                           ([70, 0], "mixed", 20, "causal-codes"),
                                                           ([40, 0], "mixed", 12, "two-passes"),
                                                           (None, "mixed", 0, "copy-region"),
                                                           (None, None, 0, "no-codes"),
                                                           ([40, 0], "mixed", 0, "replay"),
                                                           ([40, 0], "mixed", 12, "raw"),
                                                           ([40, 0], "mixed", 64, "raw")])
def test_masked_prefill_f32_matches_fp64(prompt_len, quota, tail, policy):
    from abridgekv_amd import ops
    xattn = "causal" if policy == "causal-codes" else "full"
    L = 2 if policy in ("two-passes", "copy-region") else 1
    cr = 65 if policy == "copy-region" else 0
    K = 0 if policy == "no-codes" else 16
    R = 12 if policy == "replay" else 0
    policy = "static" if policy in ("causal-codes", "two-passes", "copy-region", "no-codes", "replay") else policy
    C, N, B = 64, 4, 2
    S0 = N * (C + L * K + R) + cr
    head_quota = None if quota is None else [1 + (h * 5) % max(K, 1) for h in range(32)]
    g = torch.Generator().manual_seed(7)
    q = torch.randn((B, S0, 32, 128), generator=g, dtype=torch.float32)
    k = torch.randn((B, S0, 8, 128), generator=g, dtype=torch.float32)
    v = torch.randn((B, S0, 8, 128), generator=g, dtype=torch.float32)
    dev = torch.device("cuda")
    pl = None if prompt_len is None else torch.tensor(prompt_len, dtype=torch.int32, device=dev)
    hq = None if head_quota is None else torch.tensor(head_quota, dtype=torch.int32, device=dev)
    lse = torch.empty((B, 32, S0), dtype=torch.float32, device=dev)
    out, _ = ops.prefill_masked_attention(q.to(dev), k.to(dev), v.to(dev), C, K, N, prompt_len=pl, head_quota=hq,
                                          lse=lse, retain_tail=tail, tail_policy=policy, pause_xattn=xattn,
                                          pause_passes=L, copy_rows=cr, replay_rows=R, replay_exclude=R > 0)
    torch.cuda.synchronize()
    got_o, got_l = out.cpu().numpy(), lse.cpu().numpy()
    for b in range(B):
        raw = policy == "raw"                   # the kernels' raw policy is the oracle's separate raw-tail term
        mask = op.arith_mask(C, K, N, None if prompt_len is None else [prompt_len[b]], head_quota,
                             retain_tail=0 if raw else tail, tail_policy="static" if raw else policy,
                             pause_xattn=xattn, passes=L, copy_rows=cr, replay=R, replay_exclude=R > 0,
                             raw_tail=tail if raw else 0)
        if prompt_len is not None:
            mask = mask[0]
        ro, rl = op.masked_attention_fp64(q[b].numpy(), k[b].numpy(), v[b].numpy(), mask, 128 ** -0.5)
        assert np.abs(got_o[b] - ro).max() <= TOL
        assert np.abs(got_l[b].T - rl).max() <= TOL
