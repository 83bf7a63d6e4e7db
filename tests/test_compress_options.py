"""CompressLM's training options on the host (no GPU): pause passes, code-seed pools and code-row projections.
Layout, seeds and projections against the oracle's restatements; parameter names as the reference's state dicts
(compress_forward.py:181-222, 315-343, 397-432); the refusals."""
import types

import numpy as np
import pytest
import torch

from oracle import model as om

transformers = pytest.importorskip("transformers")


def _model():
    torch.manual_seed(0)
    cfg = transformers.Qwen3Config(vocab_size=97, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
                                   num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                                   max_position_embeddings=4096)
    return transformers.Qwen3ForCausalLM(cfg).eval()


def test_passes_layout_matches_the_oracle():
    from abridgekv_amd.compress_forward import CompressLM, rope_position_ids
    C, N, K, L = 8, 3, 4, 3
    clm = CompressLM(_model(), C, N, K, L=L)
    assert clm._pos_ids.view(-1).tolist() == list(om.rope_positions(C, N, K, "appended", passes=L))
    per = C + L * K
    assert clm.role.tolist() == [0 if j < C else (j - C) // K + 1 for _ in range(N) for j in range(per)]
    assert clm.loss_pos.nonzero().view(-1).tolist() == list(om.loss_rows(C, N, K, L))
    assert clm._code_rows.S0 == N * per
    assert clm._code_rows.slots.tolist() == [j - C for _ in range(N) for j in range(C, per)]
    # active code rows: code row p of a block keeps the full-K layout's position C + (p // K_act) K + p % K_act
    got = rope_position_ids(C, 2, K, 2, "appended", L=2).view(-1).tolist()
    assert got == [b * (C + 2 * K) + j for b in range(2) for j in list(range(C)) + [C, C + 1, C + K, C + K + 1]]
    assert clm.compress_mask(2).passes == L


def test_reference_parameter_names():
    from abridgekv_amd.compress_forward import CompressLM
    clm = CompressLM(_model(), 8, 2, 4, query_residual=True, code_kv_heads=True, gated_seg_pool=True)
    names = {n for n, _ in clm.named_parameters()}
    a = "model.model.layers.1.self_attn."
    assert {"pause", "seg_pool_gate", a + "q_proj.qres", a + "q_proj.orig.weight", a + "k_proj.orig.weight",
            a + "k_proj.code.weight", a + "v_proj.code.weight"} <= names
    pooled = CompressLM(_model(), 8, 2, 4, pool_init=True, code_q_heads=True)
    names = {n for n, _ in pooled.named_parameters()}
    assert {"pool_q", "pool_k.weight", "pool_v.weight", a + "q_proj.code.weight"} <= names
    assert float(pooled.pool_v.weight.detach().abs().max()) == 0.0        # a zero value map: an exact no-op at first
    assert torch.equal(pooled.model.model.layers[0].self_attn.q_proj.code.weight,
                       pooled.model.model.layers[0].self_attn.q_proj.orig.weight)


def test_refusals():
    from abridgekv_amd.compress_forward import CompressLM
    with pytest.raises(ValueError, match="one of them"):
        CompressLM(_model(), 8, 2, 4, query_residual=True, code_q_heads=True)
    with pytest.raises(ValueError, match="L=1"):
        CompressLM(_model(), 8, 2, 4, L=2, code_positions="bitrev")
    with pytest.raises(ValueError, match="active_code_rows"):
        CompressLM(_model(), 8, 2, 4, seg_pool=True, active_code_rows=2)
    with pytest.raises(ValueError, match="raw_tail must be in"):
        CompressLM(_model(), 8, 2, 4, raw_tail=9)
    with pytest.raises(ValueError, match="mutually exclusive"):
        CompressLM(_model(), 8, 2, 4, raw_tail=2, replay_tail=2)
    with pytest.raises(ValueError, match="no tails"):
        CompressLM(_model(), 8, 2, 4, raw_tail=2, code_positions="bitrev")
    with pytest.raises(ValueError, match="code_exclude_replay_tail"):
        CompressLM(_model(), 8, 2, 4, code_exclude_replay_tail=True)
    with pytest.raises(ValueError, match="positive"):
        CompressLM(_model(), 8, 2, 4, L=0)


@pytest.mark.parametrize("mode", ["seg", "gated", "pool", "plain", "override"])
def test_code_seeds_match_the_oracle(mode):
    from abridgekv_amd.compress_forward import code_seeds
    torch.manual_seed(1)
    B, N, C, K, d, T = 2, 3, 11, 4, 16, 2
    tok = torch.randn(B, N, C, d, dtype=torch.float64)
    clm = types.SimpleNamespace(K=K, K_act=K, code_excluded_tail=T, pause=torch.randn(K, d, dtype=torch.float64),
                                seg_pool=mode == "seg", gated_seg_pool=mode == "gated", pool_init=mode == "pool",
                                seg_pool_gate=torch.randn(K, dtype=torch.float64),
                                pool_q=torch.randn(K, d, dtype=torch.float64),
                                pool_k=torch.nn.Linear(d, d, bias=False).double(),
                                pool_v=torch.nn.Linear(d, d, bias=False).double())
    got = code_seeds(clm, tok, segment_mean=mode == "override")
    want = om.code_seeds(tok, clm.pause, K, T, segment_mean=mode in ("seg", "gated", "override"),
                         seg_gate=clm.seg_pool_gate if mode == "gated" else None,
                         pool=(clm.pool_q, clm.pool_k.weight.detach(), clm.pool_v.weight.detach())
                         if mode == "pool" else None)
    assert torch.allclose(got.expand_as(want), want, atol=1e-12)


def test_code_row_projections_match_the_oracle_rule():
    from abridgekv_amd.compress_forward import CompressLM
    C, N, K, L = 8, 2, 4, 2
    torch.manual_seed(2)
    clm = CompressLM(_model(), C, N, K, L=L, query_residual=True, code_kv_heads=True)
    attn = clm.model.model.layers[0].self_attn
    with torch.no_grad():
        attn.q_proj.qres.normal_()
        attn.k_proj.code.weight.normal_()
    S0 = N * (C + L * K)
    x = torch.randn(2, S0, 64)
    rows = torch.tensor([r for r in range(S0) if r % (C + L * K) >= C])
    slots = rows % (C + L * K) - C
    want_q = attn.q_proj.orig(x)
    want_q[:, rows] += attn.q_proj.qres[slots]
    want_k = attn.k_proj.orig(x)
    want_k[:, rows] = torch.nn.functional.linear(x[:, rows], attn.k_proj.code.weight)
    with torch.no_grad():
        assert torch.allclose(attn.q_proj(x), want_q, atol=1e-6)
        assert torch.allclose(attn.k_proj(x), want_k, atol=1e-6)
        y = torch.randn(2, S0 - 1, 64)                                 # another layout length: plain projections
        assert torch.equal(attn.q_proj(y), attn.q_proj.orig(y)) and torch.equal(attn.k_proj(y), attn.k_proj.orig(y))


def test_generator_projects_code_steps_like_the_forward():
    from abridgekv_amd.compress_forward import CompressLM
    from abridgekv_amd.gen_compress import _project
    C, K = 8, 4
    clm = CompressLM(_model(), C, 2, K, query_residual=True, code_kv_heads=True)
    attn = clm.model.model.layers[1].self_attn
    with torch.no_grad():
        attn.q_proj.qres.normal_()
        attn.v_proj.code.weight.normal_()
    x = torch.randn(1, K, 64)
    with torch.no_grad():
        assert torch.allclose(_project(attn.q_proj, x, True), attn.q_proj.orig(x) + attn.q_proj.qres[:K])
        assert torch.equal(_project(attn.q_proj, x, False), attn.q_proj.orig(x))
        assert torch.equal(_project(attn.v_proj, x, True), attn.v_proj.code(x))
        assert torch.equal(_project(attn.v_proj, x, False), attn.v_proj.orig(x))
        assert torch.equal(_project(attn.o_proj, x.repeat(1, 1, 64), True), attn.o_proj(x.repeat(1, 1, 64)))


def test_code_rows_follow_the_module_across_devices():
    """Built on one device, the code-row projections index on whatever device their input is on (a module moved
    after construction); checked here between the CPU and the meta device."""
    from abridgekv_amd.compress_forward import CompressLM
    clm = CompressLM(_model(), 8, 2, 4, query_residual=True)
    cr = clm._code_rows
    rows, slots = cr.at(torch.device("meta"))
    assert rows.device.type == "meta" and slots.device.type == "meta" and rows.shape == (2 * 4,)
    rows, _ = cr.at(torch.device("cpu"))
    assert rows.device.type == "cpu" and rows.tolist() == [8, 9, 10, 11, 20, 21, 22, 23]


@pytest.mark.parametrize("L,R", [(1, 3), (2, 2)])
def test_replay_layout_matches_the_oracle(L, R):
    """Replay rows after each block's codes (compress_forward.py:20-31, 72-88, 1044-1071): roles, replayed content
    positions, RoPE positions against the oracle's layout and the reference's closed forms."""
    from abridgekv_amd.compress_forward import CompressLM
    C, N, K = 8, 3, 4
    clm = CompressLM(_model(), C, N, K, L=L, replay_tail=R, code_exclude_replay_tail=True)
    per = C + L * K + R
    assert clm._pos_ids.view(-1).tolist() == list(om.rope_positions(C, N, K, "appended", passes=L, replay=R))
    assert clm.role.tolist() == [0 if j < C else (j - C) // K + 1 if j < C + L * K else L + 1
                                 for _ in range(N) for j in range(per)]
    cap = [b * C + j if j < C else b * C + C - R + (j - C - L * K) if j >= C + L * K else N * C
           for b in range(N) for j in range(per)]
    assert clm.content_abs_pos.tolist() == cap
    assert clm._code_rows.rows.tolist() == [b * per + j for b in range(N) for j in range(C, C + L * K)]
    assert clm.code_excluded_tail == R
    m = clm.compress_mask(1)
    assert (m.replay_rows, m.replay_exclude) == (R, True)
    with pytest.raises(ValueError, match="mutually exclusive"):
        CompressLM(_model(), C, N, K, replay_tail=2, retain_tail_kv=2)
    with pytest.raises(ValueError, match="L=1 and no tails"):
        CompressLM(_model(), C, N, K, replay_tail=2, code_positions="bitrev")


def test_raw_tail_is_the_kernels_raw_policy():
    """CompressLM(raw_tail=W) hands the kernels the "raw" policy with T = W (W = C allowed) and hides nothing from
    the codes: no excluded tail for the code seeds or the bitrev span."""
    from abridgekv_amd.compress_forward import CompressLM
    for W in (3, 8):
        clm = CompressLM(_model(), 8, 2, 4, raw_tail=W)
        m = clm.compress_mask(1)
        assert (m.retain_tail, m.tail_policy, m.replay_rows) == (W, "raw", 0)
        assert clm.raw_tail == W and clm.code_excluded_tail == 0
    m = CompressLM(_model(), 8, 2, 4, retain_tail_kv=3, retain_tail_policy="sticky").compress_mask(1)
    assert (m.retain_tail, m.tail_policy) == (3, "sticky")
