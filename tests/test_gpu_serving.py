"""The serving stress loop on the GPU: decode steps with code steps and compaction interleaved. Every row written
during the run must sit at the physical row the planner maps its logical position to (bit-exact tags), and decode
over the final cache through the loop's page tables must match the float64 oracle (2e-2, bf16; see _close for the
tagged dims)."""
import numpy as np
import pytest
import torch

from oracle import decode as od

pytestmark = pytest.mark.gpu


def _close(out, ref):
    """|out - ref| <= 2e-2 everywhere, except where the layout tags sit: the loop writes integer tags (up to 255)
    into dims 0..2 of KV head 0's V rows, so the outputs of query heads 0..3 in those dims are O(100) and carry the
    bf16 rounding of the output itself (|ref| * 2^-8, doubled for slack) on top."""
    bound = np.full(ref.shape, 2e-2)
    bound[..., :4, :3] += 2.0 ** -7 * np.abs(ref[..., :4, :3])
    return bool((np.abs(out - ref) <= bound).all()), float(np.abs(out - ref).max())


def test_serving_loop_layout_and_decode():
    from abridgekv_amd import ops
    from abridgekv_amd.serving import ServingStress
    rng = np.random.default_rng(0)
    B, C, K = 8, 64, 16
    quotas = (16, 4, 8, 4, 16, 8)
    T = rng.integers(200, 600, B)
    P = rng.integers(10, 150, B)
    s = ServingStress(T, P, layer_quotas=quotas, seed=0, C=C, K=K, growth_tokens=256, tag=True)
    s.run(150)
    s.flush()
    torch.cuda.synchronize()
    assert s.stats["decode_tokens"] > 0 and s.stats["code_steps"] >= B
    assert s.stats["moved_rows"] > 0
    assert s.check_layout() > B * 100
    # decode over the final state of one group through the loop's page tables and lengths
    g = 1
    cache = s.by_group[g][0]
    lens = s.seq_lens[g].astype(np.int32)
    q = torch.randn((B, 32, 128), generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    dev = torch.device("cuda")
    out, _ = ops.decode_attention(q.to(dev), cache, torch.from_numpy(s.tables[g]).to(dev),
                                  torch.from_numpy(lens).to(dev), 128 ** -0.5)
    torch.cuda.synchronize()
    ref, _ = od.decode_paged_fp64(q.float().numpy(), cache.float().cpu().numpy(), s.tables[g], lens, 128 ** -0.5)
    ok, err = _close(out.float().cpu().numpy(), ref)
    assert ok, err


def test_serving_loop_served_geometry():
    """Served geometry: C=512, K=256, the Qwen3-4B per-layer quotas (6 KV-cache groups, 36 layers), B=32 requests,
    run until every request has closed at least two blocks (code step + compaction each). Every row written during the
    run holds the logical position the planner maps it to; decode over the final state of the largest and the
    smallest quota group matches the float64 oracle on sampled requests."""
    from abridgekv_amd import ops
    from abridgekv_amd.serving import ServingStress
    rng = np.random.default_rng(7)
    B = 32
    T = rng.integers(2048, 6000, B)
    P = rng.integers(128, 1025, B)
    steps = 2 * 512 + 40
    s = ServingStress(T, P, seed=7, growth_tokens=steps + 64, tag=True)
    s.run(steps)
    s.flush()
    torch.cuda.synchronize()
    assert s.stats["code_steps"] >= 2 * B, s.stats
    assert s.check_layout() > B * steps
    dev = torch.device("cuda")
    for g in (0, s.G - 1):
        cache = s.by_group[g][0]
        lens = s.seq_lens[g].astype(np.int32)
        q = torch.randn((B, 32, 128), generator=torch.Generator().manual_seed(g)).to(torch.bfloat16)
        bt = torch.from_numpy(s.tables[g]).to(dev)
        out, _ = ops.decode_attention(q.to(dev), cache, bt, torch.from_numpy(lens).to(dev), 128 ** -0.5)
        torch.cuda.synchronize()
        for b in sorted({int(np.argmin(lens)), int(np.argmax(lens)), 5}):
            n = int(lens[b])
            pos = torch.arange(n, device=dev)
            rows = cache[bt[b].long()[pos // 16], :, pos % 16].float().cpu().numpy()
            ref, _ = od.decode_fp64(q[b].float().numpy(), rows[:, 0], rows[:, 1], 128 ** -0.5)
            ok, err = _close(out[b].float().cpu().numpy(), ref)
            assert ok, (g, b, err)


def _per_layer_stress(concurrent, **kw):
    """A serving loop that keeps every layer's attention output in a buffer of its own (the product shares one
    buffer between layers), so a code step that read queries already rotated by the next layer's append would show."""
    from abridgekv_amd.serving import ServingStress

    class PerLayer(ServingStress):
        def _layer_out(self, layer):
            if not hasattr(self, "_outs"):
                self._outs = [torch.zeros_like(self.out) for _ in range(self.L)]
            return self._outs[layer]

    return PerLayer(concurrent_code_step=concurrent, **kw)


@pytest.mark.parametrize("geometry", ["small", "served"])
def test_concurrent_code_step_matches_serial(geometry):
    """The code step on its own stream (forked after the layer's append, joined before the next layer's) gives every
    layer's decode and code-step rows bit-identical to the same loop with the code step after the decode on one
    stream, on every step of a run with code steps and compaction."""
    rng = np.random.default_rng(3)
    if geometry == "small":
        B, steps = 8, 140
        kw = dict(T=rng.integers(200, 600, B), P=rng.integers(10, 150, B), layer_quotas=(16, 4, 8, 4, 16, 8), C=64,
                  K=16, growth_tokens=256)
    else:
        B, steps = 16, 40
        # every request 1..8 tokens short of a block boundary, so code steps run within the first steps
        T = 512 * rng.integers(4, 10, B) - rng.integers(1, 9, B)
        kw = dict(T=T, P=rng.integers(128, 1025, B), growth_tokens=steps + 64)
    # the same key splits in both orders (their defaults differ: a quarter of the CUs beside the decode, all of them
    # after it), so the outputs can be compared bit for bit
    kw["code_target_blocks"] = 64
    a = _per_layer_stress(True, seed=5, **kw)
    b = _per_layer_stress(False, seed=5, **kw)
    code_steps = 0
    for _ in range(steps):
        ma, mb = a.step(), b.step()
        assert ma["nc"] == mb["nc"] and ma["nd"] == mb["nd"]
        torch.cuda.synchronize()
        n = ma["n_tok"]
        for layer in range(a.L):
            assert torch.equal(a._outs[layer][:n], b._outs[layer][:n]), (layer, ma["nc"])
        code_steps += int(ma["nc"] > 0)
    assert code_steps >= (4 if geometry == "small" else 2), code_steps
    assert a.stats == b.stats


def test_serving_loop_with_host_written_move_lists():
    """The loop's fallback when the planner refuses run descriptors for a step (more than eight removals of one
    request and group): every step's moves taken as host-written lists instead. Every row written during the run still
    holds the logical position the planner maps it to."""
    from abridgekv_amd.serving import ServingStress
    rng = np.random.default_rng(0)
    B = 8
    s = ServingStress(rng.integers(200, 600, B), rng.integers(10, 150, B), layer_quotas=(16, 4, 8, 4, 16, 8), seed=0,
                      C=64, K=16, growth_tokens=256, tag=True)
    planner = s.plan.planner

    def refuse(*a, **k):
        raise RuntimeError("take_move_runs failed (-2): more than 8 span removals of one request and group")

    planner.take_step_move_runs = refuse
    s.run(150)
    s.flush()
    torch.cuda.synchronize()
    assert s.stats["moved_rows"] > 0 and s.stats["code_steps"] >= B
    assert s.check_layout() > B * 100
