"""The replay tail in serving (replay_tail = R, appended code positions; the reference's default configuration) on
the CPU: the reference's own scenarios (scripts/test_compresslm_vllm_state.py:99-283, 354-361) through the product
state machine, the product machine against the oracle trace (removal calls, kept rows, code exclusion ranges,
preemption replay), and the serving visibility of every query -- the rows resident when it runs -- against the
teacher-forced mask with replay rows (oracle.prefill.arith_mask(replay=R))."""
from types import SimpleNamespace

import numpy as np
import pytest

from abridgekv_amd.config import CompressLMConfig
from abridgekv_amd.processor import (CODE, CONTENT, REPLAY, CompressLMProcessor, RequestStatus, SamplingSpec,
                                     ServingRequest)
from oracle import prefill as op
from oracle import trace as ot


def _proc(C=4, K=2, R=2, exclude=False, packed=False):
    codes = list(range(900, 900 + K))
    cfg = CompressLMConfig(enable=True, block_size=C, num_code_tokens=K, replay_tail=R,
                           code_exclude_replay_tail=exclude, packed_kv=packed, packed_kv_k_max=K)
    cfg.set_code_token_ids(codes)
    return CompressLMProcessor(cfg), codes


def run_case(prompt, generated, R=2, exclude=False, packed=False, packed_events=None):
    """The driving loop of scripts/test_compresslm_vllm_state.py:99-214 (block_size 4, two codes, raw prompt, the
    replay tail of its default); mask events are (start, end, num_computed_tokens)."""
    proc, codes = _proc(R=R, exclude=exclude, packed=packed)
    req = ServingRequest("r", prompt, SamplingSpec(max_tokens=len(generated), bad_words_token_ids=[[c] for c in codes]))
    state = proc.prepare_request(req)
    req.compresslm_state = state
    events, gi, roles = [], 0, []

    def mask_span(_rid, start, end, groups=None):
        assert 0 <= start < end <= req.num_computed_tokens
        events.append((start, end, req.num_computed_tokens))
        return SimpleNamespace(success=True, error_message=None)

    pack = None if packed_events is None else (lambda _rid, s, e: packed_events.append((s, e)))
    for _ in range(400):
        if req.status != RequestStatus.RUNNING:
            break
        count = proc.limit_num_new_tokens(req, req.num_tokens - req.num_computed_tokens)
        assert count > 0
        start = req.num_computed_tokens
        assert all(state.roles[p] == state.roles[start] for p in range(start, start + count))
        if state.roles[start] == CODE:
            assert count == 2
        roles.append(state.roles[start])
        skip = proc.should_skip_sampling(req, count)
        req.num_computed_tokens += count
        sampled = [] if skip else [generated[gi]]
        gi += 0 if skip else 1
        proc.update_after_step(req, count, sampled, mask_span, max_model_len=256, pack_code_span=pack)
    else:
        raise AssertionError("state machine did not terminate")
    assert state.visible_output_token_ids == generated and gi == len(generated)
    assert set(roles) <= {CONTENT, CODE, REPLAY}
    for block in state.blocks:
        if block.code_span is None:
            continue
        cs, ce = block.code_span
        assert req.all_token_ids[cs:ce] == codes and state.roles[cs:ce] == [CODE, CODE]
        if block.replay_positions:
            assert [req.all_token_ids[p] for p in block.replay_positions] == block.content_token_ids[-R:]
            assert all(state.roles[p] == REPLAY for p in block.replay_positions)
        if exclude:
            tail = block.content_positions[-R:]
            assert block.code_excluded_content_span == (tail[0], tail[-1] + 1)
        else:
            assert block.code_excluded_content_span is None
    prompt_pos = {p for b in state.blocks for p in b.prompt_content_positions}
    assert not any(p in prompt_pos for s, e, _ in events for p in range(s, e))
    return req, state, events, proc


def test_reference_scenarios():
    """Exact-boundary prompt: the first sampled token is held until the codes and the replay ran, then becomes the
    next content token; a multi-block prompt with a straddling block compacts; with code_exclude_replay_tail the
    blocks record the replayed rows as the codes' excluded span."""
    req, state, _, _ = run_case([10, 11, 12, 13], [20, 21, 22, 23, 24, 25])
    first_code_end = state.blocks[0].replay_positions[-1] + 1
    assert req.all_token_ids[first_code_end] == 20
    assert req.all_token_ids[:10] == [10, 11, 12, 13, 900, 901, 12, 13, 20, 21]
    _, state, events, _ = run_case([30, 31, 32, 33, 34, 35], [40, 41, 42, 43, 44, 45, 46])
    assert len(state.blocks) >= 3 and events
    run_case([70, 71, 72, 73], [80, 81, 82, 83, 84, 85], exclude=True)


def test_replay_rows_expire_one_per_next_block_content_token():
    """Block 0 = [10 | 20 21 22] (positions 0-3), codes 4-5, replay 6-7; block 1's content tokens at 8 and 9 expire
    replay rows 6 and 7 once they have run (a prompt block's replay rows too)."""
    req, state, events, _ = run_case([10], [20, 21, 22, 23, 24, 25, 26, 27])
    b0 = state.blocks[0]
    assert b0.code_span == (4, 6) and b0.replay_positions == [6, 7]
    assert (6, 7, 9) in events and (7, 8, 10) in events
    assert state.expired_replay_positions.issuperset({6, 7})
    _, state, events, _ = run_case([10, 11, 12, 13, 14], [20, 21, 22, 23, 24, 25])       # a full prompt block
    assert (6, 7, 9) in events and (7, 8, 10) in events


def test_bulk_limit_ends_content_chunks_at_replay_expiries():
    proc, _ = _proc()
    st = SimpleNamespace(roles=[CONTENT] * 8, content_to_expired_replay={3: 0}, content_to_expired_retained_tail={})
    req = SimpleNamespace(compresslm_state=st, num_computed_tokens=2, num_tokens=8)
    assert proc.limit_num_new_tokens(req, proposed=6) == 2
    st.roles = [REPLAY] * 8
    assert proc.limit_num_new_tokens(req, proposed=4) == 4              # replay runs are chunked freely


def test_packed_kv_with_replay_archives_then_removes():
    """Packed mode with a replay tail: each block's codes are archived, then its response content and codes go as
    one span after its replay rows ran; the replay rows stay until the next block's content expires them."""
    packed = []
    _, state, events, _ = run_case([10, 11, 12, 13], [20, 21, 22, 23, 24, 25], packed=True, packed_events=packed)
    b0, b1 = state.blocks[:2]
    assert packed[0] == b0.code_span and packed[1] == b1.code_span
    masks = [(s, e) for s, e, _ in events]
    assert b0.code_span in masks                                         # a prompt block: only its codes go
    assert (b1.response_content_positions[0], b1.code_span[1]) in masks
    done = {e: c for s, e, c in events}
    assert done[b0.code_span[1]] == b0.replay_positions[-1] + 1          # after the replay rows ran


def _drive(prompt_len, gen, C, K, R, exclude, preempt_at=None):
    """Product machine and oracle trace side by side (one KV-cache group); per-step records for the visibility
    check: (kept rows before the step, start, n, role)."""
    proc, codes = _proc(C, K, R, exclude)
    req = ServingRequest("r", list(range(100, 100 + prompt_len)),
                         SamplingSpec(max_tokens=gen, bad_words_token_ids=[[c] for c in codes]))
    removed = []

    def kept(upto):
        return [p for p in range(upto) if not any(s <= p < e for s, e in removed)]

    def l2p(pos, group=0):
        assert not any(s <= pos < e for s, e in removed)
        return pos - sum(e - s for s, e in removed if e <= pos)

    req.logical_to_physical = l2p
    calls = []

    def mask_span(_rid, start, end, groups=None):
        calls.append((start, end, None if groups is None else list(groups)))
        removed.append((start, end))
        return SimpleNamespace(success=True, error_message=None)

    state = proc.prepare_request(req)
    req.compresslm_state = state
    tr = ot.RequestTrace(prompt_len, gen, C, K, (K,), replay=R)
    oracle_calls, steps, preempted = [], [], False
    for i in range(4000):
        if req.status != RequestStatus.RUNNING:
            break
        if preempt_at is not None and i == preempt_at:
            proc.reset_for_preemption(state)
            tr.preempt()
            req.num_computed_tokens = 0
            removed.clear()
            preempted = True
        count = proc.limit_num_new_tokens(req, req.num_tokens - req.num_computed_tokens)
        assert count == tr.next_chunk()
        start = req.num_computed_tokens
        role = state.roles[start]
        if role == CODE and exclude:
            (ps, pe), = proc.code_excluded_physical_ranges(req, 1)
            ls, le = proc.code_excluded_logical_range(req)
            kg = kept(start)
            assert (ps, pe) == (kg.index(ls), kg.index(le - 1) + 1)
        steps.append((kept(start), start, count, role))
        skip = proc.should_skip_sampling(req, count)
        req.num_computed_tokens += count
        tr.num_computed_tokens += count
        proc.update_after_step(req, count, [] if skip else [7], mask_span, max_model_len=1 << 20)
        oracle_calls += tr.after_step(count)
        assert kept(req.num_computed_tokens) == tr.kept_positions(0)
    assert calls == oracle_calls
    assert preempt_at is None or preempted
    return state, steps


CASES = [  # prompt length, generated tokens, C, K, R, code_exclude_replay_tail, preempt at step
    (1, 40, 8, 4, 3, False, None),
    (6, 35, 8, 4, 3, True, None),
    (13, 30, 8, 4, 8, False, 23),
    (3, 40, 8, 2, 6, True, 31),
    (9, 30, 8, 4, 1, False, 17),
]


@pytest.mark.parametrize("case", CASES, ids=[f"p{c[0]}-R{c[4]}{'-x' if c[5] else ''}{'-preempt' if c[6] else ''}"
                                             for c in CASES])
def test_product_machine_matches_trace_and_serving_visibility_is_the_training_mask(case):
    """Every query of every step sees exactly its row of the teacher-forced mask with replay rows: a content or replay
    query the resident rows before the step and its chunk causally; a code query the resident rows (less the
    block's replayed content rows with code_exclude_replay_tail) and its block's codes. Logical positions are the
    mask's sequence indices (C content rows, K code rows, R replay rows per block)."""
    prompt_len, gen, C, K, R, exclude, preempt_at = case
    state, steps = _drive(prompt_len, gen, C, K, R, exclude, preempt_at)
    assert len(state.compacted_block_ids) >= 3
    N = len(state.blocks)
    per = C + K + R
    mask = op.arith_mask(C, K, N, prompt_len=[prompt_len], replay=R, replay_exclude=exclude)[0]
    checked = 0
    for kept, start, n, role in steps:
        before = set(kept)
        for p in range(start, start + n):
            if role in (CONTENT, REPLAY):
                got = before | set(range(start, p + 1))
            else:
                blk = p // per
                ex = set(range(blk * per + C - R, blk * per + C)) if exclude else set()
                got = (before - ex) | set(range(start, start + K))
            want = set(np.nonzero(mask[p])[0].tolist())
            assert got == want, (p, role, sorted(got ^ want))
            checked += 1
    assert checked > 50


def test_bulk_decode_replay_respects_replay_expiries():
    """update_after_decode_steps (a known history replayed in bulk) gives the state of one-token steps when the
    stretch starts after the block's replay-expiring content tokens, and refuses a stretch that would expire a replay
    row (a removal it cannot issue)."""
    def drive(bulk):
        proc, codes = _proc(C=8, K=2, R=3)
        req = ServingRequest("r", [5], SamplingSpec(max_tokens=60, bad_words_token_ids=[[c] for c in codes]))
        state = proc.prepare_request(req)
        req.compresslm_state = state
        events = []

        def mask_span(_rid, s, e, groups=None):
            events.append((s, e))
            return SimpleNamespace(success=True, error_message=None)

        tok = 40
        while len(state.visible_output_token_ids) < 30:
            start = req.num_computed_tokens
            role = state.roles[start]
            if role == CONTENT and bulk and req.num_tokens == start + 1:
                blk = state.current_block
                room = 8 - len(blk.content_positions)
                if room > 1 and len(blk.content_positions) > 3:   # the newest token is not computed yet
                    ids = list(range(tok, tok + room - 1))
                    tok += len(ids)
                    req.num_computed_tokens += len(ids)
                    proc.update_after_decode_steps(req, ids, 1 << 20)
                    continue
            count = proc.limit_num_new_tokens(req, req.num_tokens - start)
            skip = proc.should_skip_sampling(req, count)
            req.num_computed_tokens += count
            sampled = [] if skip else [tok]
            tok += 0 if skip else 1
            proc.update_after_step(req, count, sampled, mask_span, max_model_len=1 << 20)
        return state, events

    bulk_state, bulk_events = drive(True)
    one_state, one_events = drive(False)
    assert bulk_state.visible_output_token_ids == one_state.visible_output_token_ids
    assert bulk_state.roles == one_state.roles and bulk_events == one_events

    proc, codes = _proc(C=8, K=2, R=3)
    req = ServingRequest("r", [5] * 8, SamplingSpec(max_tokens=60, bad_words_token_ids=[[c] for c in codes]))
    state = proc.prepare_request(req)
    req.compresslm_state = state
    ok = SimpleNamespace(success=True, error_message=None)
    while state.blocks[0].replay_positions == [] or req.num_computed_tokens <= state.blocks[0].replay_positions[-1]:
        n = proc.limit_num_new_tokens(req, req.num_tokens - req.num_computed_tokens)
        skip = proc.should_skip_sampling(req, n)
        req.num_computed_tokens += n
        proc.update_after_step(req, n, [] if skip else [40], lambda *_a, **_k: ok, max_model_len=1 << 20)
    req.num_computed_tokens += 2
    with pytest.raises(RuntimeError, match="replayed decode step"):
        proc.update_after_decode_steps(req, [41, 42], 1 << 20)
