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
