"""The product state machine (abridgekv_amd.processor) and config against the oracle restatement and the reference's
own CPU test scenarios (scripts/test_compresslm_physical_quotas.py:68-208)."""
from types import SimpleNamespace

import numpy as np
import pytest

from abridgekv_amd.config import CompressLMConfig, layer_index
from abridgekv_amd.planner import KVPlanner
from abridgekv_amd.processor import CODE, CompressLMProcessor, RequestStatus, SamplingSpec, ServingRequest
from oracle import layout as ol
from oracle import trace as ot

CODES = [900, 901, 902, 903]


def make(quotas=(4, 2, 1, 2), C=4, K=4):
    cfg = CompressLMConfig(replay_tail=0, enable=True, block_size=C, num_code_tokens=K, code_positions="bitrev",
                           layer_code_quotas=quotas, physical_layer_quotas=True)
    cfg.set_code_token_ids(CODES[:K] if K <= 4 else list(range(900, 900 + K)))
    proc = CompressLMProcessor(cfg)
    proc.set_group_quotas(quotas)
    return cfg, proc


def test_config_positions_match_oracle_and_validate():
    cfg = CompressLMConfig(replay_tail=0, code_positions="bitrev", enable=True, block_size=512, num_code_tokens=256,
                           layer_code_quotas=ol.PERLAYER_MEAN128_QUOTAS, physical_layer_quotas=True)
    assert np.array_equal(cfg.bitrev_code_offsets(), ol.bitrev_code_offsets(256, 512))
    logical = np.arange(5 * 768)
    assert np.array_equal(cfg.bitrev_rope_positions(logical), ol.bitrev_rope_positions(logical, 512, 256))
    groups, gq = cfg.kv_cache_groups(36)
    assert (groups, gq) == ol.quota_groups(ol.PERLAYER_MEAN128_QUOTAS)
    names = [[f"model.layers.{l}.self_attn.attn" for l in layers] for layers in groups]
    assert cfg.kv_group_quotas(names) == tuple(gq)
    assert layer_index("model.layers.12.self_attn.attn") == 12 and layer_index("lm_head") is None
    with pytest.raises(ValueError):
        cfg.kv_group_quotas([["model.layers.0.a", "model.layers.1.a"]])         # mixes quotas 256 and 64
    for bad in (dict(layer_code_quotas=(300,)), dict(replay_tail=16), dict(num_passes=2), dict(raw_prompt=False),
                dict(num_code_tokens=96), dict(physical_layer_quotas=True)):
        with pytest.raises(ValueError):
            CompressLMConfig(enable=True, block_size=512, code_positions="bitrev",
                             replay_tail=bad.pop("replay_tail", 0), num_code_tokens=bad.pop("num_code_tokens", 256),
                             **bad)
    # the reference's defaults: appended code positions and a replay tail of 16 (config/compresslm.py:19-44); per-layer
    # quotas below K need the bitrev layout, and the replay tail excludes the retained one
    default = CompressLMConfig(enable=True)
    assert (default.code_positions, default.replay_tail, default.code_excluded_tail) == ("appended", 16, 0)
    assert CompressLMConfig(enable=True, code_exclude_replay_tail=True).code_excluded_tail == 16
    for bad in (dict(layer_code_quotas=(64,) * 36), dict(retain_tail_kv=8), dict(raw_tail=4),
                dict(replay_tail=513), dict(code_exclude_replay_tail=True, replay_tail=0),
                dict(packed_kv=True, packed_kv_k_max=128, code_exclude_replay_tail=True)):
        with pytest.raises(ValueError):
            CompressLMConfig(enable=True, **bad)


def run_reference_scenario(proc, request, mask_span, generated):
    """The driving loop of scripts/test_compresslm_physical_quotas.py:100-121."""
    state = request.compresslm_state
    gi, code_steps = 0, 0
    for _ in range(400):
        if request.status != RequestStatus.RUNNING:
            break
        proposed = request.num_tokens - request.num_computed_tokens
        count = proc.limit_num_new_tokens(request, proposed)
        role = state.roles[request.num_computed_tokens]
        if role == CODE:
            code_steps += 1
        skip = proc.should_skip_sampling(request, count)
        yield count, role
        request.num_computed_tokens += count
        sampled = []
        if not skip:
            sampled = [generated[gi]]
            gi += 1
        proc.update_after_step(request, count, sampled, mask_span, max_model_len=256)
    else:
        raise AssertionError("did not terminate")
    assert gi == len(generated) and code_steps >= 2


def test_group_removals_keep_codes_prefix_recording_mask():
    """Reference test scenario with the reference's recording mask_span: each compacted block keeps exactly codes[:q]
    in group q and no response content; code_physical_spans exposes only the block being coded."""
    quotas = (4, 2, 1, 2)
    _, proc = make(quotas)
    req = ServingRequest("r", [11, 12, 13, 14, 15, 16], SamplingSpec(max_tokens=13, bad_words_token_ids=[[c] for c in CODES]))
    removed = [[] for _ in quotas]

    def l2p(pos, group=0):
        assert not any(s <= pos < e for s, e in removed[group])
        return pos - sum(e - s for s, e in removed[group] if e <= pos)

    req.logical_to_physical = l2p

    def mask_span(_rid, start, end, groups=None):
        for g in (range(len(quotas)) if groups is None else groups):
            assert not any(s < end and start < e for s, e in removed[g])
            removed[g].append((start, end))
        return SimpleNamespace(success=True, error_message=None)

    req.compresslm_state = proc.prepare_request(req)
    generated = list(range(21, 34))
    for count, role in run_reference_scenario(proc, req, mask_span, generated):
        for g in range(len(quotas)):
            phys = [t for i, t in enumerate(req.all_token_ids) if not any(s <= i < e for s, e in removed[g])]
            spans = proc.code_physical_spans(req, g)
            for ps, pe in spans:
                assert pe - ps == 4 and phys[ps:pe] == CODES
            if role == CODE:
                assert len(spans) == 1
    state = req.compresslm_state
    for g, q in enumerate(quotas):
        for block in state.blocks:
            if block.block_id in state.compacted_block_ids and block.code_span:
                cs, ce = block.code_span
                kept = [req.all_token_ids[p] for p in range(cs, ce) if not any(s <= p < e for s, e in removed[g])]
                assert kept == CODES[:q]
                assert all(any(s <= p < e for s, e in removed[g]) for p in block.response_content_positions)
    n = len(state.compacted_block_ids)
    for g, q in enumerate(quotas):
        assert sum(e - s for s, e in removed[g]) - sum(e - s for s, e in removed[0]) == n * (4 - q)


@pytest.mark.parametrize("prompt_len,gen", [(6, 13), (1, 30), (9, 25), (16, 9)])
def test_calls_match_oracle_trace_and_drive_the_planner(prompt_len, gen):
    """The product machine issues the same compaction calls as the oracle trace, and driving the native planner with
    them keeps its per-group layouts equal to the brute-force kept positions."""
    quotas = (4, 2, 1, 2)
    _, proc = make(quotas, C=8, K=4)
    planner = KVPlanner(2048, len(quotas), 2)
    req = ServingRequest(7, list(range(100, 100 + prompt_len)),
                         SamplingSpec(max_tokens=gen, bad_words_token_ids=[[c] for c in CODES]), planner=planner)
    planner.add_request(7)
    req.compresslm_state = proc.prepare_request(req)
    tr = ot.RequestTrace(prompt_len, gen, 8, 4, quotas)
    calls_p, calls_o = [], []

    def mask_span(rid, start, end, groups=None):
        calls_p.append((start, end, None if groups is None else list(groups)))
        return planner.mask_token_span(rid, start, end, groups)

    for step in range(500):
        if req.status != RequestStatus.RUNNING:
            break
        n = proc.limit_num_new_tokens(req, req.num_tokens - req.num_computed_tokens)
        assert n == tr.next_chunk()
        skip = proc.should_skip_sampling(req, n)
        assert planner.allocate_slots(7, n) is not None
        req.num_computed_tokens += n
        planner.set_num_computed_tokens(7, req.num_computed_tokens)
        tr.num_computed_tokens += n
        proc.update_after_step(req, n, [] if skip else [500 + step], mask_span, max_model_len=10_000)
        calls_o.extend(tr.after_step(n))
        planner.take_step_outputs()
        for g in range(len(quotas)):
            active = req.num_computed_tokens - planner.compacted_counts(7)[g]
            phys = [planner.physical_to_logical(7, x, g) for x in range(active)]
            assert phys == tr.kept_positions(g)
    assert calls_p == [(s, e, g) for s, e, g in calls_o]
    assert tr.finished and req.status == RequestStatus.FINISHED_LENGTH_CAPPED


def test_preemption_bounds_code_spans():
    """scripts/test_compresslm_physical_quotas.py:170-208 restated: after a preemption the logical structure survives
    but the KV does not; logical_limit admits exactly the blocks whose codes are back in the KV."""
    _, proc = make((4, 2, 1, 2))
    req = ServingRequest("r", [11, 12, 13, 14, 15, 16], SamplingSpec(max_tokens=13, bad_words_token_ids=[[c] for c in CODES]))
    state = proc.prepare_request(req)
    req.compresslm_state = state
    state.blocks = [SimpleNamespace(block_id=i, code_span=(100 * i + 20, 100 * i + 24), response_content_positions=[])
                    for i in range(4)]
    proc.reset_for_preemption(state)
    req.num_computed_tokens = 0
    assert len(proc.code_physical_spans(req, 0)) == 4
    for limit, expected in [(0, 0), (23, 0), (24, 1), (124, 2), (224, 3), (324, 4), (10_000, 4)]:
        got = proc.code_physical_spans(req, 0, limit)
        assert len(got) == expected and all(e <= limit for _, e in got)


def test_request_validation():
    _, proc = make()
    with pytest.raises(ValueError):
        proc.prepare_request(ServingRequest("a", [1, 2], SamplingSpec(bad_words_token_ids=[])))
    with pytest.raises(ValueError):
        proc.prepare_request(ServingRequest("a", [], SamplingSpec(bad_words_token_ids=[[c] for c in CODES])))
    with pytest.raises(ValueError):
        CompressLMProcessor(CompressLMConfig(replay_tail=0, code_positions="bitrev",
                                             enable=True, block_size=4, num_code_tokens=4))


@pytest.mark.parametrize("change,message", [
    (dict(prompt_token_ids=None), "requires prompt token IDs"),
    (dict(prompt_embeds=[[0.0]]), "does not support prompt_embeds"),
    (dict(pooling_params=object()), "only supports generation requests"),
    (dict(sampling=None), "requires sampling parameters"),
    (dict(frequency_penalty=0.5), "frequency_penalty=0"),
    (dict(presence_penalty=-0.1), "presence_penalty=0"),
    (dict(repetition_penalty=1.1), "repetition_penalty=1"),
    (dict(stop=["\n\n"]), "not stop strings"),
    (dict(min_tokens=3), "min_tokens=0"),
    (dict(logprobs=2), "only available in debug mode"),
    (dict(prompt_logprobs=0), "does not support prompt logprobs"),
    (dict(use_structured_output=True), "does not support structured output"),
])
def test_request_refusals_match_the_reference(change, message):
    """Each request the reference's prepare_request refuses (processor.py:42-80) is refused with its message; the
    same request with the field at its default is accepted."""
    _, proc = make()
    bans = [[c] for c in CODES]
    spec = {k: v for k, v in change.items() if k in SamplingSpec.__dataclass_fields__}
    req_kw = {k: v for k, v in change.items() if k not in spec and k not in ("prompt_token_ids", "sampling")}
    sampling = None if "sampling" in change else SamplingSpec(bad_words_token_ids=bans, **spec)
    prompt = change.get("prompt_token_ids", [1, 2, 3])
    req = ServingRequest("a", prompt, sampling, **req_kw)
    if sampling is None:
        req.sampling_params = None
    with pytest.raises(ValueError, match=message):
        proc.prepare_request(req)
    ok = ServingRequest("b", [1, 2, 3], SamplingSpec(bad_words_token_ids=bans))
    assert proc.prepare_request(ok).pending_prompt_index == 3


def test_logprobs_are_allowed_in_debug_mode():
    cfg = CompressLMConfig(replay_tail=0, code_positions="bitrev",
                           enable=True, block_size=4, num_code_tokens=2, debug=True)
    cfg.set_code_token_ids([90, 91])
    proc = CompressLMProcessor(cfg)
    req = ServingRequest("a", [1, 2], SamplingSpec(bad_words_token_ids=[[90], [91]], logprobs=1))
    assert proc.prepare_request(req).pending_prompt_index == 2


def test_config_json_round_trip_and_schedule_loading(tmp_path):
    """compresslm_config.json written as the reference's exporter writes it, read back the way its serving entry
    points read it, with per-layer quotas from the reference's schedule file (tests/golden)."""
    import json
    from pathlib import Path

    from abridgekv_amd.config import load_layer_quotas, load_quota_rows
    from abridgekv_amd.workloads import QWEN3_4B_LAYER_QUOTAS

    sched = Path(__file__).parent / "golden" / "sched_trunc_perlayer_mean128.json"
    rows = load_quota_rows(sched)
    assert len(rows) == 36 and all(len(r) == 8 for r in rows)
    assert load_layer_quotas(sched) == QWEN3_4B_LAYER_QUOTAS
    assert sum(load_layer_quotas(sched)) == 4608

    cfg = CompressLMConfig(replay_tail=0, code_positions="bitrev", enable=True, block_size=512, num_code_tokens=256)
    cfg.set_code_token_ids(list(range(1000, 1256)))
    path = cfg.write_json(tmp_path)
    meta = json.loads(path.read_text())
    assert meta["code_positions"] == "bitrev" and meta["code_token_ids"][:2] == [1000, 1001]
    assert set(meta) == {"enable", "block_size", "num_code_tokens", "num_passes", "pause_xattn", "raw_prompt",
                         "raw_tail", "replay_tail", "code_positions", "retain_tail_kv", "retain_tail_policy",
                         "code_exclude_replay_tail", "code_token_format", "code_token_ids"}
    meta["code_rows_of_k_max"] = 256                       # exporter provenance, not a config field
    path.write_text(json.dumps(meta))
    back = CompressLMConfig.from_json(tmp_path, layer_quotas_path=sched, physical_layer_quotas=True)
    assert back.layer_code_quotas == QWEN3_4B_LAYER_QUOTAS and back.uses_physical_layer_quotas
    assert back.code_token_ids == list(range(1000, 1256))
    groups, gq = back.kv_cache_groups(36)
    assert gq == [256, 64, 64, 128, 128, 128] and groups[0] == [0, 15, 18, 20, 21, 24]

    bad = tmp_path / "bad.json"
    bad.write_text(json.dumps([[64] * 7 + [128]]))
    with pytest.raises(ValueError):
        load_layer_quotas(bad)
    bad.write_text(json.dumps({"other": 1}))
    with pytest.raises(ValueError):
        load_quota_rows(bad)


def _state_tuple(req):
    st = req.compresslm_state
    return (req.num_computed_tokens, list(req.all_token_ids), list(req._output_token_ids), req.status,
            st.roles, st.position_to_block, st.visible_output_token_ids, st.held_sampled_token, st.current_block_id,
            st.pending_prompt_index, sorted(st.compacted_block_ids), st.worker_token_ids_dirty,
            [(b.block_id, b.content_positions, b.content_token_ids, b.prompt_content_positions,
              b.response_content_positions, b.code_span) for b in st.blocks])


@pytest.mark.parametrize("seed", range(8))
def test_bulk_decode_replay_equals_per_token_steps(seed):
    """update_after_decode_steps (a stretch of one-token decode steps at once, as the history builder replays them)
    leaves exactly the state of calling update_after_step once per step; stretches that reach the block end or hit a
    stop token take the per-token path (and a stop raises)."""
    rng = np.random.default_rng(seed)
    C, K = 16, 4
    _, proc = make(quotas=(4, 2, 1, 2), C=C, K=K)
    sp = SamplingSpec(bad_words_token_ids=[[c] for c in CODES], stop_token_ids=(77,))
    prompt = rng.integers(1, 50, int(rng.integers(1, 3 * C))).tolist()
    reqs = [ServingRequest(i, prompt, sp, eos_token_id=99) for i in range(2)]
    calls = [[], []]
    for i, r in enumerate(reqs):
        r.compresslm_state = proc.prepare_request(r)

    def rec(i):
        def mask(rid, s, e, groups=None):
            calls[i].append((s, e, groups))
            return SimpleNamespace(success=True, error_message=None)
        return mask

    for _ in range(60):
        a, b = reqs
        start = a.num_computed_tokens
        pending = a.num_tokens - start
        st = a.compresslm_state
        if st.roles[start] == CODE or pending > 1:          # code run or prompt chunk: both step normally
            n = proc.limit_num_new_tokens(a, pending)
            skip = proc.should_skip_sampling(a, n)
            tok = [] if skip else [int(rng.integers(1, 50))]
            for i, r in enumerate(reqs):
                r.num_computed_tokens += n
                proc.update_after_step(r, n, tok, rec(i), 1 << 20)
        else:
            # at most up to the step that computes the block's last content token (it stages the codes)
            m = int(rng.integers(1, C - len(st.current_block.content_positions) + 2))
            ids = rng.integers(1, 50, m).tolist()
            for tok in ids:
                b.num_computed_tokens += 1
                proc.update_after_step(b, 1, [tok], rec(1), 1 << 20)
            a.num_computed_tokens += m
            proc.update_after_decode_steps(a, ids, 1 << 20)
        assert _state_tuple(a) == _state_tuple(b)
        assert calls[0] == calls[1]
    assert calls[0], "no block was compacted"
    r = reqs[0]
    while r.compresslm_state.roles[r.num_computed_tokens] == CODE or r.num_tokens - r.num_computed_tokens > 1:
        n = proc.limit_num_new_tokens(r, r.num_tokens - r.num_computed_tokens)
        skip = proc.should_skip_sampling(r, n)
        r.num_computed_tokens += n
        proc.update_after_step(r, n, [] if skip else [5], rec(0), 1 << 20)
    if len(r.compresslm_state.current_block.content_positions) + 2 > C:     # keep the stop inside the block
        return
    r.num_computed_tokens += 2
    with pytest.raises(RuntimeError, match="stopped"):
        proc.update_after_decode_steps(r, [5, 77], 1 << 20)


def test_block_removal_spans_order():
    """The removals of a closed block: response content in every group, then code slots [q, K) per quota q < K in
    ascending q; packed KV removes content and codes as one span."""
    from abridgekv_amd.processor import CompressLMBlock
    _, proc = make(quotas=(4, 2, 1, 2), C=8, K=4)
    blk = CompressLMBlock(0, content_positions=list(range(8)), prompt_content_positions=[0, 1, 2],
                          response_content_positions=list(range(3, 8)), code_span=(8, 12))
    assert proc.block_removal_spans(blk) == [(3, 8, None), (9, 12, [2]), (10, 12, [1, 3])]
    blk.response_content_positions = []
    assert proc.block_removal_spans(blk) == [(9, 12, [2]), (10, 12, [1, 3])]
    blk.response_content_positions = [3, 5]
    with pytest.raises(RuntimeError, match="contiguous"):
        proc.block_removal_spans(blk)
