"""Decode parity at the full saturated serving size: B=256 sequences of up to 32K logical tokens, the Qwen3-4B quota
groups' page tables from the compaction planner, one layer per group. Every sequence is checked for finite output and
LSE; a sample of sequences (shortest, longest, two seeded) is compared with the float64 oracle over the rows gathered
from the same cache (max-abs <= 2e-2 for outputs and LSE)."""
import numpy as np
import pytest
import torch

from oracle import decode as od

pytestmark = pytest.mark.gpu
TOL = 2e-2


def test_saturated_batch_matches_oracle_on_a_sample():
    from abridgekv_amd import ops, workloads
    T, P = workloads.saturated_decode_lengths(256, seed=0)
    st = workloads.build_decode_state(T, P, seed=0)
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(0)
    cache = torch.empty(ops.kv_cache_shape(st.num_pages), dtype=torch.bfloat16, device=dev)
    cache.normal_(generator=gen)
    rng = np.random.default_rng(0)
    scale = 128 ** -0.5
    for g in (0, len(st.groups) - 1):
        sl = st.seq_lens[g]
        bt = torch.from_numpy(st.block_tables[g]).to(dev)
        q = torch.randn((256, 32, 128), generator=gen, device=dev).to(torch.bfloat16)
        lse = torch.empty((256, 32), dtype=torch.float32, device=dev)
        max_pages = int(-(-int(sl.max()) // 16))
        out, _ = ops.decode_attention(q, cache, bt, torch.from_numpy(sl).to(dev), scale, max_pages=max_pages, lse=lse)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all() and torch.isfinite(lse).all(), f"group {g}"
        pick = sorted({int(np.argmin(sl)), int(np.argmax(sl)), *rng.integers(0, 256, 2).tolist()})
        for b in pick:
            n = int(sl[b])
            pos = torch.arange(n, device=dev)
            pages = bt[b].long()[pos // 16]
            rows = cache[pages, :, pos % 16].float().cpu().numpy()           # [n, 2, 8, 128]
            ref_o, ref_l = od.decode_fp64(q[b].float().cpu().numpy(), rows[:, 0], rows[:, 1], scale)
            assert np.abs(out[b].float().cpu().numpy() - ref_o).max() <= TOL, f"group {g} seq {b} ({n} rows)"
            assert np.abs(lse[b].cpu().numpy() - ref_l).max() <= TOL, f"group {g} seq {b}"


def test_full_model_decode_b64_matches_oracle_on_a_sample():
    """The full-model decode workload: B=64, 512-token prompt (its block also gets codes), 32 generated closed
    blocks compressed to the 256/128/64 per-layer quotas, open block U[1, 511]; page tables from the compaction
    planner. One layer of every KV-cache group (the auto split the bench picks for it); all outputs and LSE finite;
    the shortest, the longest and two seeded sequences per group against the float64 oracle."""
    from abridgekv_amd import ops, workloads
    T, P = workloads.full_model_decode_lengths(64, seed=0)
    st = workloads.build_decode_state(T, P, seed=0)
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(3)
    cache = torch.empty(ops.kv_cache_shape(st.num_pages), dtype=torch.bfloat16, device=dev)
    cache.normal_(generator=gen)
    rng = np.random.default_rng(3)
    scale = 128 ** -0.5
    W = st.block_tables[0].shape[1]
    ws = ops.decode_workspace(64, W, 32, device=dev)
    for g in range(len(st.groups)):
        sl = st.seq_lens[g]
        q_l = st.group_quotas[g]
        # rows = 512 prompt rows + 33 code sets of q_l rows + the open block's L = T - 33 * 512 rows
        assert np.array_equal(sl, 512 + 33 * q_l + (T - 33 * 512)), f"group {g}"
        bt = torch.from_numpy(st.block_tables[g]).to(dev)
        q = torch.randn((64, 32, 128), generator=gen, device=dev).to(torch.bfloat16)
        lse = torch.empty((64, 32), dtype=torch.float32, device=dev)
        max_pages = int(-(-int(sl.max()) // 16))
        out, _ = ops.decode_attention(q, cache, bt, torch.from_numpy(sl).to(dev), scale, max_pages=max_pages, lse=lse,
                                      split_pages=ops.auto_split_pages(sl), workspace=ws)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all() and torch.isfinite(lse).all(), f"group {g}"
        pick = sorted({int(np.argmin(sl)), int(np.argmax(sl)), *rng.integers(0, 64, 2).tolist()})
        for b in pick:
            n = int(sl[b])
            pos = torch.arange(n, device=dev)
            pages = bt[b].long()[pos // 16]
            rows = cache[pages, :, pos % 16].float().cpu().numpy()
            ref_o, ref_l = od.decode_fp64(q[b].float().cpu().numpy(), rows[:, 0], rows[:, 1], scale)
            assert np.abs(out[b].float().cpu().numpy() - ref_o).max() <= TOL, f"group {g} seq {b} ({n} rows)"
            assert np.abs(lse[b].cpu().numpy() - ref_l).max() <= TOL, f"group {g} seq {b}"
