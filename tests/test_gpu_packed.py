"""Per-head packed code pages on the GPU against the oracle (oracle/packed.py): the capture kernel bit-exact, the
packed decode and multi-query attention within the bf16 bound (max-abs <= 2e-2 for outputs and LSE), and the
sidecar end to end."""
import numpy as np
import pytest
import torch

from oracle import packed as opk

pytestmark = pytest.mark.gpu
TOL = 2e-2
K = 16
SCHED = [(1, 16, 3, 5, 2, 7, 4, 16), (16,) * 8, (8, 8, 1, 1, 12, 3, 9, 2)]


def _bf(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16)


def _f64(t):
    return t.float().cpu().numpy().astype(np.float64)


def _setup(seed, num_pages=400):
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    caches = [torch.randn((num_pages, 2, 16, 8, 128), generator=g).to(torch.bfloat16) for _ in SCHED]
    return rng, caches


def test_capture_is_bit_exact():
    from abridgekv_amd import ops
    rng, caches = _setup(0)
    dev = torch.device("cuda")
    dc = [c.to(dev) for c in caches]
    rows = [sum(r) for r in SCHED]
    pools = [torch.zeros((20, 2, n, 128), dtype=torch.bfloat16, device=dev) for n in rows]
    caps = []
    for i in range(5):
        table = rng.permutation(np.arange(1, 400))[:8].astype(np.int32)
        start = int(rng.integers(0, 8 * 16 - K + 1))
        caps.append((table, start, int(rng.integers(0, 20))))
    caps = list({c[2]: c for c in caps}.values())         # one capture per destination page
    bt = torch.from_numpy(np.stack([c[0] for c in caps])).to(dev)
    meta = torch.tensor([c[1] for c in caps] + [c[2] for c in caps], dtype=torch.int32, device=dev)
    ops.packed_capture(dc, pools, torch.tensor(rows, dtype=torch.int32, device=dev),
                       torch.tensor(SCHED, dtype=torch.int32, device=dev), bt, meta[: len(caps)], meta[len(caps):])
    torch.cuda.synchronize()
    for l, row in enumerate(SCHED):
        got = pools[l].cpu()
        for table, start, page in caps:
            ref = opk.capture(caches[l].float().numpy(), table, start, K, row)
            assert np.array_equal(got[page].float().numpy(), ref), f"layer {l} page {page}"


def _packed_state(rng, caches, counts, pool_pages=64):
    """Pools filled by the oracle's capture from random code spans, and per-sequence page lists."""
    pools, pages = [], []
    free = list(rng.permutation(pool_pages))
    for n in counts:
        pages.append([int(free.pop()) for _ in range(n)])
    srcs = {}
    for seq in pages:
        for p in seq:
            srcs[p] = (rng.permutation(np.arange(1, caches[0].shape[0]))[:4].astype(np.int32), int(rng.integers(0, 48)))
    for l, row in enumerate(SCHED):
        pool = np.zeros((pool_pages, 2, sum(row), 128), dtype=np.float32)
        for p, (t, s) in srcs.items():
            pool[p] = opk.capture(caches[l].float().numpy(), t, s, K, row)
        pools.append(pool)
    return pools, pages


def _table(pages):
    width = max(1, max(len(p) for p in pages))
    t = np.zeros((len(pages), width), dtype=np.int32)
    for i, p in enumerate(pages):
        t[i, : len(p)] = p
    return t, np.asarray([len(p) for p in pages], dtype=np.int32)


@pytest.mark.parametrize("layer", [0, 1, 2])
def test_decode_packed_matches_oracle(layer):
    from abridgekv_amd import ops
    rng, caches = _setup(10 + layer)
    lens = [0, 1, 17, 300, 1100, 37]
    counts = [3, 0, 1, 7, 2, 40]
    pools, pages = _packed_state(rng, caches, counts)
    row = SCHED[layer]
    need = [-(-n // 16) for n in lens]
    perm = rng.permutation(np.arange(1, 400))
    bt = np.zeros((len(lens), max(need)), dtype=np.int32)
    at = 0
    for i, n in enumerate(need):
        bt[i, :n] = perm[at: at + n]
        at += n
    g = torch.Generator().manual_seed(99)
    q = torch.randn((len(lens), 32, 128), generator=g).to(torch.bfloat16)
    dev = torch.device("cuda")
    table, count = _table(pages)
    lse = torch.empty((len(lens), 32), dtype=torch.float32, device=dev)
    out, _ = ops.decode_attention_packed(q.to(dev), caches[layer].to(dev), torch.from_numpy(bt).to(dev),
                                         torch.tensor(lens, dtype=torch.int32, device=dev),
                                         _bf(pools[layer]).to(dev), row, torch.from_numpy(table).to(dev),
                                         torch.from_numpy(count).to(dev), 128 ** -0.5, lse=lse)
    torch.cuda.synchronize()
    cf = caches[layer].float().numpy()
    for i in range(len(lens)):
        ro, rl = opk.packed_attention_fp64(_f64(q[i:i + 1]), [pools[layer][p] for p in pages[i]], row, cf, bt[i],
                                           lens[i], 1, True, K, 128 ** -0.5)
        go, gl = _f64(out[i]), lse[i].cpu().numpy()
        assert np.abs(go - ro[0]).max() <= TOL, f"seq {i}"
        live = np.isfinite(rl[0])
        assert np.abs(gl[live] - rl[0][live]).max(initial=0) <= TOL
        assert np.all(np.isneginf(gl[~live])) and np.all(go[~live] == 0)


@pytest.mark.parametrize("tail", [0, 23])
def test_multi_query_packed_matches_oracle(tail):
    """A causal prompt chunk, a code step (K queries, non-causal, paged keys < prefix + q_h per head; with a static
    tail, the block's last rows before the codes hidden) and a chunk of a request with no packed pages in one
    launch."""
    from abridgekv_amd import ops
    rng, caches = _setup(20)
    layer = 0
    row = SCHED[layer]
    reqs = [(70, 400, True), (K, 300, False), (130, 130, True)]      # (query_len, seq_len, causal)
    counts = [5, 9, 0]
    pools, pages = _packed_state(rng, caches, counts)
    need = [-(-sl // 16) for _, sl, _ in reqs]
    perm = rng.permutation(np.arange(1, 400))
    bt = np.zeros((len(reqs), max(need)), dtype=np.int32)
    at = 0
    for i, n in enumerate(need):
        bt[i, :n] = perm[at: at + n]
        at += n
    qsl = np.concatenate([[0], np.cumsum([r[0] for r in reqs])])
    g = torch.Generator().manual_seed(5)
    q = torch.randn((int(qsl[-1]), 32, 128), generator=g).to(torch.bfloat16)
    dev = torch.device("cuda")
    table, count = _table(pages)
    sls = np.asarray([r[1] for r in reqs])
    ql = np.asarray([r[0] for r in reqs])
    lse = torch.empty((int(qsl[-1]), 32), dtype=torch.float32, device=dev)
    excluded = [(sl - n - tail, sl - n) if tail and not causal else None for n, sl, causal in reqs]
    out, _ = ops.paged_prefill_attention_packed(q.to(dev), caches[layer].to(dev), torch.from_numpy(bt).to(dev), qsl,
                                                sls - ql, sls, [r[2] for r in reqs], _bf(pools[layer]).to(dev), row,
                                                torch.from_numpy(table).to(dev), torch.from_numpy(count).to(dev),
                                                int(count.max()), scale=128 ** -0.5, lse=lse,
                                                excluded=excluded if tail else None)
    torch.cuda.synchronize()
    cf = caches[layer].float().numpy()
    for i, (n, sl, causal) in enumerate(reqs):
        ro, rl = opk.packed_attention_fp64(_f64(q[qsl[i]: qsl[i + 1]]), [pools[layer][p] for p in pages[i]], row, cf,
                                           bt[i], sl, n, causal, K, 128 ** -0.5, excluded=excluded[i])
        assert np.abs(_f64(out[qsl[i]: qsl[i + 1]]) - ro).max() <= TOL, f"request {i}"
        assert np.abs(lse[qsl[i]: qsl[i + 1]].cpu().numpy() - rl).max() <= TOL, f"request {i}"


def test_sidecar_capture_then_decode():
    from abridgekv_amd.packed_kv import PackedKVLayout, PackedKVSidecar
    rng, caches = _setup(30)
    dev = torch.device("cuda")
    layout = PackedKVLayout.from_schedule(SCHED, num_layers=3, num_kv_heads=8, k_max=K)
    dc = [c.to(dev) for c in caches]
    side = PackedKVSidecar(layout, dc, pool_pages=32, max_pages_per_request=8)
    tables = {r: rng.permutation(np.arange(1, 400))[:20].astype(np.int32) for r in ("a", "b")}
    caps = {"a": [0, 40, 100], "b": [16]}
    for r, starts in caps.items():
        for s in starts:
            side.capture(r, physical_start=s, physical_end=s + K, block_ids=tables[r].tolist())
    assert side.allocated_bytes == 4 * layout.bytes_per_block(head_size=128, element_size=2)
    lens = [250, 300]
    bt = torch.from_numpy(np.stack([tables["a"], tables["b"]])).to(dev)
    g = torch.Generator().manual_seed(3)
    q = torch.randn((2, 32, 128), generator=g).to(torch.bfloat16)
    out = torch.empty((2, 32, 128), dtype=torch.bfloat16, device=dev)
    for layer, row in enumerate(SCHED):
        side.attend(layer, q.to(dev), dc[layer], bt, [0, 1, 2], lens, True, out, request_ids=("a", "b"),
                    scale=128 ** -0.5)
        torch.cuda.synchronize()
        cf = caches[layer].float().numpy()
        for i, r in enumerate(("a", "b")):
            pages = [opk.capture(cf, tables[r], s, K, row) for s in caps[r]]
            ro, _ = opk.packed_attention_fp64(_f64(q[i:i + 1]), pages, row, cf, tables[r], lens[i], 1, True, K,
                                              128 ** -0.5)
            assert np.abs(_f64(out[i]) - ro[0]).max() <= TOL, f"layer {layer} request {r}"
    side.free("a")
    assert side.request_pages("a") == [] and len(side._free) == 32 - 1


def test_decode_packed_wide_quotas_matches_oracle():
    """Head quotas of 32 and more, some not multiples of 32 (the side kernel then takes a 32-row chunk's two packed
    pages by readlane, and chunks straddle page boundaries), up to 40 packed pages per sequence so that splits span
    many pages; packed pools filled at random."""
    from abridgekv_amd import ops
    row = (32, 48, 64, 100, 128, 160, 200, 256)
    rng = np.random.default_rng(31)
    g = torch.Generator().manual_seed(31)
    cache = torch.randn((400, 2, 16, 8, 128), generator=g).to(torch.bfloat16)
    lens = [1, 17, 300, 1100, 37, 520]
    counts = [3, 0, 1, 7, 40, 12]
    pool_pages = 70
    pool = torch.randn((pool_pages, 2, sum(row), 128), generator=g).to(torch.bfloat16)
    free = list(rng.permutation(pool_pages))
    pages = [[int(free.pop()) for _ in range(n)] for n in counts]
    need = [-(-n // 16) for n in lens]
    perm = rng.permutation(np.arange(1, 400))
    bt = np.zeros((len(lens), max(need)), dtype=np.int32)
    at = 0
    for i, n in enumerate(need):
        bt[i, :n] = perm[at: at + n]
        at += n
    q = torch.randn((len(lens), 32, 128), generator=g).to(torch.bfloat16)
    dev = torch.device("cuda")
    table, count = _table(pages)
    lse = torch.empty((len(lens), 32), dtype=torch.float32, device=dev)
    out, _ = ops.decode_attention_packed(q.to(dev), cache.to(dev), torch.from_numpy(bt).to(dev),
                                         torch.tensor(lens, dtype=torch.int32, device=dev), pool.to(dev), row,
                                         torch.from_numpy(table).to(dev), torch.from_numpy(count).to(dev),
                                         128 ** -0.5, lse=lse)
    torch.cuda.synchronize()
    cf, pf = cache.float().numpy(), pool.float().numpy()
    for i in range(len(lens)):
        ro, rl = opk.packed_attention_fp64(_f64(q[i:i + 1]), [pf[p] for p in pages[i]], row, cf, bt[i], lens[i], 1,
                                           True, 256, 128 ** -0.5)
        go, gl = _f64(out[i]), lse[i].cpu().numpy()
        assert np.abs(go - ro[0]).max() <= TOL, f"seq {i}"
        assert np.abs(gl - rl[0]).max() <= TOL
