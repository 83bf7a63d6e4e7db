"""Pins of the dense teacher-forced model oracle (oracle/model.py) on a random tiny model in float64."""
import numpy as np
import pytest
import torch

from oracle import layout as ol
from oracle import model as om

transformers = pytest.importorskip("transformers")


def tiny_model(layers=2, seed=0, dtype=torch.float64):
    torch.manual_seed(seed)
    cfg = transformers.Qwen3Config(vocab_size=97, hidden_size=64, intermediate_size=96, num_hidden_layers=layers,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=16,
                                   max_position_embeddings=4096, rope_parameters={"rope_theta": 1e6,
                                                                                  "rope_type": "default"})
    cfg._attn_implementation = "eager"
    return transformers.Qwen3ForCausalLM(cfg).to(dtype).eval()


def test_rope_positions_closed_form():
    C, N, K = 16, 3, 8
    bitrev = om.rope_positions(C, N, K, "bitrev")
    offs = ol.bitrev_code_offsets(K, C)
    for b in range(N):
        assert list(bitrev[b * (C + K): b * (C + K) + C]) == list(range(b * C, b * C + C))
        assert list(bitrev[b * (C + K) + C: (b + 1) * (C + K)]) == list(b * C + offs)
    assert list(om.rope_positions(C, N, K, "appended")) == list(range(N * (C + K)))
    # a static tail of 5: code rows spread over [0, 11) -- the reference's own check (test_compresslm_vllm_state.py:
    # 349-352, C=8, K=4, T=2: offsets < 6, distinct, the first 0)
    tail = om.rope_positions(C, N, K, "bitrev", span=C - 5)[C: C + K] - 0
    assert tail.max() < C - 5 and len(set(tail.tolist())) == K and tail[0] == 0
    assert list(ol.bitrev_code_offsets(4, 8, 6)) == [0, 3, 1, 4]


@pytest.mark.parametrize("code_positions", ["appended", "bitrev"])
def test_one_block_content_logits_equal_causal_forward(code_positions):
    model = tiny_model()
    C, K = 16, 4
    ids = torch.randint(0, 97, (2, 1, C))
    pause = torch.randn(K, 64, dtype=torch.float64) * 0.05
    got = om.dense_loss_logits(model, pause, ids, C, 1, K, code_positions)
    with torch.no_grad():
        ref = model(input_ids=ids.view(2, C), position_ids=torch.arange(C).view(1, C)).logits[:, : C - 1]
    # HF eager attention takes its softmax in float32 even for a float64 model: ~1e-7 apart, a wrong mask or
    # position would be ~1e-2 apart
    assert torch.allclose(got, ref.reshape(-1, 97).double(), atol=1e-6)


def test_full_quotas_equal_no_quotas_and_quotas_matter():
    model = tiny_model()
    C, N, K = 16, 3, 8
    ids = torch.randint(0, 97, (2, N, C))
    pause = torch.randn(K, 64, dtype=torch.float64) * 0.05
    base = om.dense_loss_logits(model, pause, ids, C, N, K, "bitrev", prompt_len=[5, 20])
    full = om.dense_loss_logits(model, pause, ids, C, N, K, "bitrev", prompt_len=[5, 20],
                                layer_head_quota=np.full((2, 4), K))
    assert torch.allclose(base, full, atol=1e-12)
    small = om.dense_loss_logits(model, pause, ids, C, N, K, "bitrev", prompt_len=[5, 20],
                                 layer_head_quota=np.full((2, 4), 2))
    assert not torch.allclose(base, small, atol=1e-6)


def test_rope_positions_with_passes():
    C, N, K = 8, 3, 4
    assert list(om.rope_positions(C, N, K, "appended", passes=3)) == list(range(N * (C + 3 * K)))
    assert list(om.loss_rows(C, N, K, passes=2)) == [b * (C + 2 * K) + j for b in range(N) for j in range(C - 1)]
    assert list(om.rope_positions(C, N, K, "appended", passes=2, replay=3)) == list(range(N * (C + 2 * K + 3)))
    assert list(om.loss_rows(C, N, K, 1, 3)) == [b * (C + K + 3) + j for b in range(N) for j in range(C - 1)]


@pytest.mark.parametrize("exclude", [False, True])
def test_replay_rows_change_later_blocks_only(exclude):
    """Replay rows follow a block's codes: the first block's content never sees them (its logits are the model's
    causal forward), and the next block's content does."""
    model = tiny_model()
    C, N, K, R = 12, 2, 4, 3
    ids = torch.randint(0, 97, (2, N, C))
    pause = torch.randn(K, 64, dtype=torch.float64) * 0.05
    got = om.dense_loss_logits(model, pause, ids, C, N, K, replay=R, replay_exclude=exclude)
    with torch.no_grad():
        ref = model(input_ids=ids[:, 0], position_ids=torch.arange(C).view(1, C)).logits[:, : C - 1]
    per_seq = N * (C - 1)
    for b in range(2):
        assert torch.allclose(got[b * per_seq: b * per_seq + C - 1], ref[b].double(), atol=1e-6)
    plain = om.dense_loss_logits(model, pause, ids, C, N, K)
    later = slice(C - 1, per_seq)
    assert not torch.allclose(got[later], plain[later], atol=1e-6)


def _code_proj(model, K, L, seed, scale=0.05):
    g = torch.Generator().manual_seed(seed)
    out = []
    for layer in model.model.layers:
        a = layer.self_attn
        dq, dk = a.q_proj.out_features, a.k_proj.out_features
        out.append({"qres": torch.randn(L * K, dq, generator=g, dtype=torch.float64) * scale,
                    "k": (a.k_proj.weight.detach() + torch.randn(dk, 64, generator=g, dtype=torch.float64) * scale,
                          None)})
    return out


@pytest.mark.parametrize("passes", [1, 2, 3])
def test_one_block_content_logits_ignore_codes_passes_seeds_and_projections(passes):
    """The content rows of a single block precede its code rows and never see them, so neither the passes, the
    seeds nor the code rows' projections may change the content logits: they equal the model's causal forward."""
    model = tiny_model()
    C, K = 12, 4
    ids = torch.randint(0, 97, (2, 1, C))
    pause = torch.randn(K, 64, dtype=torch.float64) * 0.05
    seeds = torch.randn(2, 1, K, 64, dtype=torch.float64)
    got = om.dense_loss_logits(model, pause, ids, C, 1, K, "appended", passes=passes, seeds=seeds,
                               code_proj=_code_proj(model, K, passes, 3), pause_xattn="causal")
    with torch.no_grad():
        ref = model(input_ids=ids.view(2, C), position_ids=torch.arange(C).view(1, C)).logits[:, : C - 1]
    assert torch.allclose(got, ref.reshape(-1, 97).double(), atol=1e-6)


def test_identity_code_projections_change_nothing_and_real_ones_reach_later_blocks_only():
    model = tiny_model()
    C, N, K, L = 12, 3, 4, 2
    ids = torch.randint(0, 97, (2, N, C))
    pause = torch.randn(K, 64, dtype=torch.float64) * 0.05
    base = om.dense_loss_logits(model, pause, ids, C, N, K, passes=L)
    same = []
    for layer in model.model.layers:
        a = layer.self_attn
        same.append({"qres": torch.zeros(L * K, a.q_proj.out_features, dtype=torch.float64),
                     "q": (a.q_proj.weight.detach(), None), "k": (a.k_proj.weight.detach(), None),
                     "v": (a.v_proj.weight.detach(), None)})
    assert torch.allclose(om.dense_loss_logits(model, pause, ids, C, N, K, passes=L, code_proj=same), base,
                          atol=1e-12)
    moved = om.dense_loss_logits(model, pause, ids, C, N, K, passes=L, code_proj=_code_proj(model, K, L, 5))
    per_seq = N * (C - 1)
    for b in range(2):
        first = slice(b * per_seq, b * per_seq + C - 1)                  # block 0's content: no codes before it
        later = slice(b * per_seq + C - 1, (b + 1) * per_seq)
        assert torch.allclose(moved[first], base[first], atol=1e-12)
        assert not torch.allclose(moved[later], base[later], atol=1e-6)
    # the passes matter: a second pass changes what later blocks read
    one = om.dense_loss_logits(model, pause, ids, C, N, K, passes=1)
    assert not torch.allclose(one, base, atol=1e-6)


def test_code_seeds_pools():
    torch.manual_seed(0)
    B, N, C, K, d = 2, 2, 10, 3, 8
    tok = torch.randn(B, N, C, d, dtype=torch.float64)
    pause = torch.randn(K, d, dtype=torch.float64)
    # segment means: K runs of (C - T) // K rows of the first C - T rows, written out by hand
    T = 2
    got = om.code_seeds(tok, pause, K, excluded_tail=T, segment_mean=True)
    seg = (C - T) // K
    for b in range(B):
        for n in range(N):
            for k in range(K):
                rows = [tok[b, n, k * seg + i] for i in range(seg)]
                assert torch.allclose(got[b, n, k], pause[k] + sum(rows) / seg)
    gate = torch.tensor([0.0, 1.0, -2.0], dtype=torch.float64)
    gated = om.code_seeds(tok, pause, K, excluded_tail=T, segment_mean=True, seg_gate=gate)
    assert torch.allclose(gated[:, :, 0], pause[0].expand(B, N, d))
    assert torch.allclose(gated[:, :, 2] - pause[2], -2.0 * (got[:, :, 2] - pause[2]))
    # fewer content rows than codes: every code takes the block mean
    few = om.code_seeds(tok[:, :, :2], torch.zeros(4, d, dtype=torch.float64), 4, segment_mean=True)
    assert torch.allclose(few, tok[:, :, :2].mean(2, keepdim=True).expand(B, N, 4, d))
    # pooling: a zero value map leaves the seeds; a one-hot pooling picks one row's value
    eye = torch.eye(d, dtype=torch.float64)
    pq = torch.randn(K, d, dtype=torch.float64)
    assert torch.allclose(om.code_seeds(tok, pause, K, pool=(pq, eye, torch.zeros(d, d, dtype=torch.float64))),
                          pause.expand(B, N, K, d))
    basis = torch.zeros(B, N, C, d, dtype=torch.float64)
    for i in range(C):
        basis[:, :, i, i % d] = 1.0 / (1 + i // d)                  # rows 0..7: e_0..e_7; rows 8, 9: e_0 / 2, e_1 / 2
    pick = torch.zeros(K, d, dtype=torch.float64)
    for k in range(K):
        pick[k, 2 * k] = 400.0                                       # code k's query aligns with row 2k
    wv = torch.randn(d, d, dtype=torch.float64)
    pooled = om.code_seeds(basis, torch.zeros(K, d, dtype=torch.float64), K, pool=(pick, eye, wv))
    for k in range(K):
        assert torch.allclose(pooled[:, :, k], (wv @ basis[0, 0, 2 * k]).expand(B, N, d), atol=1e-9)
