"""Attention backend on the GPU: one mixed step (decodes, a causal prompt chunk, code steps of two quotas) with the
K/V append, checked against fp64 attention under the reference-format masks; the custom-mask entry; graph capture
of decode steps (tolerance: max-abs <= 2e-2 for bf16 outputs)."""
import numpy as np
import pytest
import torch

from abridgekv_amd import backend as bk
from abridgekv_amd import ops
from oracle import decode as od
from oracle import masks as om

pytestmark = pytest.mark.gpu
TOL = 2e-2
K_CODES = 256


def _step(seed):
    """Requests (query_len, seq_len after the step, code span or None) of one group, decodes first."""
    rng = np.random.default_rng(seed)
    reqs = [(1, int(rng.integers(1, 900)), None) for _ in range(3)]
    reqs.append((150, 150 + 333, None))                          # prompt chunk after 333 cached rows
    for res in (700, 64):
        reqs.append((K_CODES, res + K_CODES, (res, res + K_CODES)))
    return reqs


def _tables(reqs, num_pages, rng):
    need = [-(-sl // 16) for _, sl, _ in reqs]
    assert sum(need) < num_pages
    perm = rng.permutation(np.arange(1, num_pages))
    tables = np.zeros((len(reqs), max(need)), np.int32)
    at = 0
    for r, n in enumerate(need):
        tables[r, :n] = perm[at: at + n]
        at += n
    return tables


def _slots(reqs, tables):
    out = []
    for r, (ql, sl, _) in enumerate(reqs):
        pos = np.arange(sl - ql, sl)
        out.append(tables[r, pos // 16].astype(np.int64) * 16 + pos % 16)
    return np.concatenate(out)


@pytest.mark.parametrize("quota", [64, 256])
def test_mixed_step_matches_masked_oracle(quota):
    reqs = _step(quota)
    rng = np.random.default_rng(1)
    tables = _tables(reqs, 400, rng)
    g = torch.Generator().manual_seed(quota)
    cache = torch.randn((400, 2, 16, 8, 128), generator=g).to(torch.bfloat16)
    T = sum(r[0] for r in reqs)
    q = torch.randn((T, 32 * 128), generator=g).to(torch.bfloat16)
    k_new = torch.randn((T, 8 * 128), generator=g).to(torch.bfloat16)
    v_new = torch.randn((T, 8 * 128), generator=g).to(torch.bfloat16)
    slots = _slots(reqs, tables)

    dev = torch.device("cuda")
    qsl = np.concatenate([[0], np.cumsum([r[0] for r in reqs])])
    sls = [r[1] for r in reqs]
    limits = bk.code_step_key_limits(qsl, sls, [r[2] for r in reqs], quota, K_CODES)
    builder = bk.AbridgeMetadataBuilder(max_num_seqs=8, max_pages=tables.shape[1], device=dev)
    md = builder.build(qsl, sls, torch.from_numpy(tables).to(dev), torch.from_numpy(slots).to(dev),
                       code_key_limit=limits)
    impl = bk.AbridgeAttentionImpl()
    cache_d = cache.to(dev)
    out = torch.empty((T, 32 * 128), dtype=torch.bfloat16, device=dev)
    impl.forward(None, q.to(dev), k_new.to(dev), v_new.to(dev), cache_d, md, out)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(T, 32, 128)

    # expected: the cache after the append (numpy), fp64 attention under the reference's flat mask per request
    cf = cache.float().numpy().copy()
    pages, offs = slots // 16, slots % 16
    cf[pages, 0, offs] = k_new.float().numpy().reshape(T, 8, 128)
    cf[pages, 1, offs] = v_new.float().numpy().reshape(T, 8, 128)
    assert torch.equal(cache_d.cpu()[pages, 0, offs], k_new.reshape(T, 8, 128))
    qf = q.float().numpy().reshape(T, 32, 128)
    for r, (ql, sl, span) in enumerate(reqs):
        m = om.request_mask(ql, sl, [span] if span else [], None, quota, K_CODES, causal=span is None)
        ro, _ = om.masked_paged_attention_fp64(qf[qsl[r]: qsl[r + 1]], cf, tables[r], sl, m, 128 ** -0.5)
        assert np.abs(got[qsl[r]: qsl[r + 1]] - ro).max() <= TOL, f"request {r}"

    # the same step through the reference's flat custom mask -> limits
    flat = np.concatenate([om.request_mask(ql, sl, [span] if span else [], None, quota, K_CODES,
                                           causal=span is None).reshape(-1) for ql, sl, span in reqs])
    lim2, causal2 = bk.limits_from_custom_mask(torch.from_numpy(flat), qsl, sls)
    code2 = np.where(np.diff(qsl) > 1, np.where(causal2, bk.NOT_CODE, lim2), bk.NOT_CODE)
    md2 = builder.build(qsl, sls, md.block_table, md.slot_mapping, code_key_limit=code2)
    out2 = torch.empty_like(out)
    layer = type("Layer", (), {})()
    bk.attach(layer, impl)
    bk.maybe_override_attention(layer, q.to(dev), cache_d, md2, out2)
    torch.cuda.synchronize()
    assert torch.equal(out2, out)


def test_decode_steps_replay_in_a_graph():
    """Capture append + decode once; replay with new inputs three times, each checked against an eager run."""
    dev = torch.device("cuda")
    rng = np.random.default_rng(7)
    B = 16
    sls = rng.integers(1, 3000, B).tolist()
    reqs = [(1, s, None) for s in sls]
    tables = _tables(reqs, 3200, rng)
    slots = torch.from_numpy(_slots(reqs, tables)).to(dev)
    g = torch.Generator().manual_seed(8)
    base = torch.randn((3200, 2, 16, 8, 128), generator=g).to(torch.bfloat16).to(dev)
    builder = bk.AbridgeMetadataBuilder(max_num_seqs=B, max_pages=tables.shape[1], device=dev)
    md = builder.build(np.arange(B + 1), sls, torch.from_numpy(tables).to(dev), slots)
    impl = bk.AbridgeAttentionImpl()
    q_s = torch.zeros((B, 32 * 128), dtype=torch.bfloat16, device=dev)
    k_s = torch.zeros((B, 8 * 128), dtype=torch.bfloat16, device=dev)
    v_s = torch.zeros((B, 8 * 128), dtype=torch.bfloat16, device=dev)
    out_s = torch.zeros((B, 32 * 128), dtype=torch.bfloat16, device=dev)
    cache_g = base.clone()
    impl.forward(None, q_s, k_s, v_s, cache_g, md, out_s)         # warm up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        impl.forward(None, q_s, k_s, v_s, cache_g, md, out_s)
    for it in range(3):
        q = torch.randn((B, 32 * 128), generator=g).to(torch.bfloat16).to(dev)
        k = torch.randn((B, 8 * 128), generator=g).to(torch.bfloat16).to(dev)
        v = torch.randn((B, 8 * 128), generator=g).to(torch.bfloat16).to(dev)
        q_s.copy_(q)
        k_s.copy_(k)
        v_s.copy_(v)
        graph.replay()
        cache_e = base.clone()
        out_e = impl.forward(None, q, k, v, cache_e, md)
        torch.cuda.synchronize()
        assert torch.equal(out_s, out_e), f"replay {it}"
        assert torch.equal(cache_g, cache_e), f"replay {it}"
    ref = od.decode_paged_fp64(q.float().cpu().numpy().reshape(B, 32, 128), cache_e.float().cpu().numpy(), tables,
                               sls, ops.default_scale())[0]
    assert np.abs(out_s.float().cpu().numpy().reshape(B, 32, 128) - ref).max() <= TOL
