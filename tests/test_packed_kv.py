"""Per-head packed code pages on the CPU: the layout API (compresslm_packed_kv.py:12-155) against the oracle, the
oracle's pins, the packed-mode config validation (config/compresslm.py:145-190) and the state machine's packed
events (the reference's own scenario, scripts/test_compresslm_vllm_state.py:283-302)."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from abridgekv_amd.config import CompressLMConfig
from abridgekv_amd.packed_kv import PackedKVLayout
from abridgekv_amd.processor import CODE, CompressLMProcessor, RequestStatus, SamplingSpec, ServingRequest
from oracle import decode as od
from oracle import masks as om
from oracle import packed as opk


def test_layout_validation_matches_reference_errors():
    with pytest.raises(ValueError, match="k_max must be positive"):
        PackedKVLayout(quotas=((1,),), k_max=0)
    with pytest.raises(ValueError, match="non-empty"):
        PackedKVLayout(quotas=(), k_max=2)
    with pytest.raises(ValueError, match="equal length"):
        PackedKVLayout(quotas=((1, 2), (1,)), k_max=2)
    with pytest.raises(ValueError, match=r"must be in \[1, 2\]"):
        PackedKVLayout(quotas=((1, 3),), k_max=2)
    with pytest.raises(ValueError, match="layers; model has"):
        PackedKVLayout.from_schedule([[1, 1]], num_layers=2, num_kv_heads=2, k_max=2)
    with pytest.raises(ValueError, match="row widths"):
        PackedKVLayout.from_schedule([[1, 1], [1]], num_layers=2, num_kv_heads=2, k_max=2)
    with pytest.raises(ValueError, match="dimensions must be positive"):
        PackedKVLayout.from_schedule(None, num_layers=0, num_kv_heads=2, k_max=2)
    uniform = PackedKVLayout.from_schedule(None, num_layers=3, num_kv_heads=2, k_max=4)
    assert uniform.quotas == ((4, 4),) * 3 and uniform.storage_ratio == 1.0


def test_layout_geometry_and_hand_worked_page():
    L = PackedKVLayout(quotas=((1, 2), (2, 2)), k_max=2)
    assert L.offsets == ((0, 1, 3), (0, 2, 4))
    assert L.packed_slots_per_layer == (3, 4) and L.packed_slots == 7 and L.dense_slots == 8
    assert L.storage_ratio == 7 / 8
    assert L.bytes_per_block(head_size=128, element_size=2) == 2 * 7 * 128 * 2
    assert L.dense_bytes_per_block(head_size=128, element_size=2) == 2 * 8 * 128 * 2
    with pytest.raises(ValueError):
        L.bytes_per_block(head_size=0, element_size=2)
    # dense[kv, slot, head, d] = 1000 kv + 100 slot + 10 head + d
    dense = np.fromfunction(lambda a, b, c, d: 1000 * a + 100 * b + 10 * c + d, (2, 2, 2, 3))
    page = opk.pack((1, 2), dense)
    # layer 0: head 0 keeps slot 0; head 1 keeps slots 0, 1 -> rows (s0 h0), (s0 h1), (s1 h1)
    assert page[0, :, 0].tolist() == [0, 10, 110] and page[1, :, 0].tolist() == [1000, 1010, 1110]
    got = L.pack_layer(0, torch.from_numpy(dense)).numpy()
    assert np.array_equal(got, page)
    back = L.unpack_layer(0, torch.from_numpy(page), fill_value=-1.0).numpy()
    assert np.array_equal(back, opk.unpack((1, 2), 2, page, fill=-1.0))
    assert np.array_equal(back[:, 0], dense[:, 0]) and np.array_equal(back[:, 1, 1], dense[:, 1, 1])
    assert np.all(back[:, 1, 0] == -1.0)
    with pytest.raises(ValueError):
        L.pack_layer(0, torch.zeros(2, 3, 2, 3))
    with pytest.raises(ValueError):
        L.unpack_layer(1, torch.from_numpy(page))


def test_oracle_round_trip_random_schedules():
    rng = np.random.default_rng(0)
    for _ in range(20):
        k_max = int(rng.integers(1, 9))
        row = tuple(int(x) for x in rng.integers(1, k_max + 1, size=8))
        dense = rng.standard_normal((2, k_max, 8, 16))
        page = opk.pack(row, dense)
        assert page.shape == (2, sum(row), 16)
        back = opk.unpack(row, k_max, page, fill=np.nan)
        for h, q in enumerate(row):
            assert np.array_equal(back[:, :q, h], dense[:, :q, h]) and np.all(np.isnan(back[:, q:, h]))


def _paged(rng, seq_len, pages_total, extra_rows=0):
    need = -(-(seq_len + extra_rows) // 16)
    table = rng.permutation(np.arange(1, pages_total))[:need]
    cache = rng.standard_normal((pages_total, 2, 16, 8, 32))
    return cache, table


def test_oracle_uniform_quota_equals_plain_attention():
    """Equal quotas q in every head: the side rows are just more keys, so the packed attention equals the plain
    attention over [q code rows of every captured block | paged rows] (decode, causal chunk and code step)."""
    rng = np.random.default_rng(1)
    K, q = 4, 3
    row = (q,) * 8
    seq_len = 70
    cache, table = _paged(rng, seq_len, 40)
    # two captured blocks taken from other pages of the same cache
    cap_tables = [rng.permutation(np.arange(1, 40))[:1] for _ in range(2)]
    pages = [opk.capture(cache, t, 5, K, row) for t in cap_tables]
    mk, mv = od.paged_rows(cache, table, seq_len)
    scale = 32 ** -0.5
    for query_len, causal in [(1, True), (5, True), (K, False)]:
        qr = rng.standard_normal((query_len, 32, 32))
        got, got_l = opk.packed_attention_fp64(qr, pages, row, cache, table, seq_len, query_len, causal, K, scale)
        for h in range(8):                 # plain keys of head h: its side rows in page order, then paged rows
            sk = np.concatenate([p[0, h * q:(h + 1) * q] for p in pages])
            sv = np.concatenate([p[1, h * q:(h + 1) * q] for p in pages])
            keys = np.concatenate([sk, mk[:, h]])
            vals = np.concatenate([sv, mv[:, h]])
            prefix = seq_len - query_len
            for i in range(query_len):
                if causal:
                    lim = prefix + i + 1
                else:
                    lim = prefix + q
                n = sk.shape[0] + lim
                for g in range(4):
                    o, l = od.decode_fp64(qr[i, 4 * h + g][None], keys[:n, None], vals[:n, None], scale)
                    assert np.allclose(got[i, 4 * h + g], o[0], atol=1e-12)
                    assert np.isclose(got_l[i, 4 * h + g], l[0], atol=1e-12)


def test_oracle_heads_depend_only_on_their_quota():
    rng = np.random.default_rng(2)
    K = 8
    mixed = (1, 8, 3, 5, 2, 7, 4, 6)
    seq_len = 40
    cache, table = _paged(rng, seq_len, 30)
    cap = [rng.permutation(np.arange(1, 30))[:1] for _ in range(3)]
    qr = rng.standard_normal((K, 32, 32))
    for causal, query_len in [(False, K), (True, 1)]:
        got, _ = opk.packed_attention_fp64(qr[:query_len], [opk.capture(cache, t, 0, K, mixed) for t in cap], mixed,
                                           cache, table, seq_len, query_len, causal, K, 0.2)
        for h, qh in enumerate(mixed):
            uni = (qh,) * 8
            ref, _ = opk.packed_attention_fp64(qr[:query_len], [opk.capture(cache, t, 0, K, uni) for t in cap], uni,
                                               cache, table, seq_len, query_len, causal, K, 0.2)
            assert np.allclose(got[:, 4 * h:4 * h + 4], ref[:, 4 * h:4 * h + 4], atol=1e-12)


def test_oracle_code_step_without_pages_is_the_code_mask():
    """No captured block: a code step is the ordinary code-step mask with limit prefix + q_h (oracle.masks)."""
    rng = np.random.default_rng(3)
    K, q = 4, 2
    seq_len = 50
    cache, table = _paged(rng, seq_len, 10)
    qr = rng.standard_normal((K, 32, 32))
    got, got_l = opk.packed_attention_fp64(qr, [], (q,) * 8, cache, table, seq_len, K, False, K, 0.3)
    m = om.request_mask(K, seq_len, [(seq_len - K, seq_len)], None, q, K, causal=False)
    ref, ref_l = om.masked_paged_attention_fp64(qr, cache, table, seq_len, m, 0.3)
    assert np.allclose(got, ref, atol=1e-12) and np.allclose(got_l, ref_l, atol=1e-12)
    ex = (seq_len - K - 7, seq_len - K)                    # the block's static tail, just before its codes
    got, got_l = opk.packed_attention_fp64(qr, [], (q,) * 8, cache, table, seq_len, K, False, K, 0.3, excluded=ex)
    m = om.request_mask(K, seq_len, [(seq_len - K, seq_len)], ex, q, K, causal=False)
    ref, ref_l = om.masked_paged_attention_fp64(qr, cache, table, seq_len, m, 0.3)
    assert np.allclose(got, ref, atol=1e-12) and np.allclose(got_l, ref_l, atol=1e-12)
    assert not np.allclose(got, opk.packed_attention_fp64(qr, [], (q,) * 8, cache, table, seq_len, K, False, K,
                                                          0.3)[0])


def test_packed_config_validation():
    ok = CompressLMConfig(replay_tail=0, code_positions="bitrev",
                          enable=True, block_size=4, num_code_tokens=2, packed_kv=True, packed_kv_k_max=2,
                          packed_kv_quotas=((1, 2),))
    assert ok.uses_packed_kv and ok.packed_layout(1, 2).quotas == ((1, 2),)
    with pytest.raises(ValueError, match="packed_kv_k_max"):
        CompressLMConfig(replay_tail=0, code_positions="bitrev",
                         enable=True, block_size=4, num_code_tokens=2, packed_kv=True)
    with pytest.raises(ValueError, match="must be in"):
        CompressLMConfig(replay_tail=0, code_positions="bitrev",
                         enable=True, block_size=4, num_code_tokens=2, packed_kv=True, packed_kv_k_max=2,
                         packed_kv_quotas=((3,),))
    with pytest.raises(ValueError, match="must not be empty"):
        CompressLMConfig(replay_tail=0, code_positions="bitrev",
                         enable=True, block_size=4, num_code_tokens=2, packed_kv=True, packed_kv_k_max=2,
                         packed_kv_quotas=((),))
    with pytest.raises(ValueError, match="mutually exclusive"):
        CompressLMConfig(replay_tail=0, code_positions="bitrev",
                         enable=True, block_size=4, num_code_tokens=2, packed_kv=True, packed_kv_k_max=2,
                         layer_code_quotas=(1, 2))


def _run_packed(prompt, generated):
    """The driving loop of scripts/test_compresslm_vllm_state.py:100-209 with packed_kv=True, K_max=2."""
    cfg = CompressLMConfig(replay_tail=0, code_positions="bitrev",
                           enable=True, block_size=4, num_code_tokens=2, packed_kv=True, packed_kv_k_max=2)
    cfg.set_code_token_ids([900, 901])
    proc = CompressLMProcessor(cfg)
    req = ServingRequest("r", prompt, SamplingSpec(max_tokens=len(generated), bad_words_token_ids=[[900], [901]]))
    state = proc.prepare_request(req)
    req.compresslm_state = state
    masks, events = [], []

    def mask_span(_rid, start, end, groups=None):
        assert 0 <= start < end <= req.num_computed_tokens
        masks.append((start, end))
        return SimpleNamespace(success=True, error_message=None)

    gi = 0
    for _ in range(200):
        if req.status != RequestStatus.RUNNING:
            break
        count = proc.limit_num_new_tokens(req, req.num_tokens - req.num_computed_tokens)
        role = state.roles[req.num_computed_tokens]
        if role == CODE:
            assert count == 2
        skip = proc.should_skip_sampling(req, count)
        req.num_computed_tokens += count
        sampled = [] if skip else [generated[gi]]
        gi += 0 if skip else 1
        proc.update_after_step(req, count, sampled, mask_span, max_model_len=256,
                               pack_code_span=lambda _rid, s, e: events.append((s, e)))
    assert state.visible_output_token_ids == generated
    return state, masks, events


def test_packed_state_machine_archives_then_removes():
    """scripts/test_compresslm_vllm_state.py:283-302: each complete code chunk is archived before both its code rows
    and the response content it summarizes are removed."""
    state, masks, events = _run_packed([10, 11, 12, 13], [20, 21, 22, 23, 24, 25])
    b0, b1 = state.blocks[0], state.blocks[1]
    assert events[0] == b0.code_span and b0.code_span in masks
    assert events[1] == b1.code_span
    assert (b1.response_content_positions[0], b1.code_span[1]) in masks
    # every archived block leaves no code or response row resident
    for b in state.blocks:
        if b.block_id in state.compacted_block_ids:
            removed = [p for s, e in masks for p in range(s, e)]
            assert all(p in removed for p in range(*b.code_span))
            assert all(p in removed for p in b.response_content_positions)
