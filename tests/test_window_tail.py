"""The window retained tails (retain_tail_kv = T with retain_tail_policy "rolling" or "sticky") on the CPU: the
reference's own scenarios (scripts/test_compresslm_vllm_state.py:357-486) through the product state machine, the
product machine against the oracle trace (removal calls, kept rows, code exclusion ranges, preemption replay), and
the serving visibility of every query -- the rows resident when it runs -- against the teacher-forced mask of the
same policy (oracle.prefill.arith_mask), for all three policies."""
from types import SimpleNamespace

import numpy as np
import pytest

from abridgekv_amd.config import CompressLMConfig
from abridgekv_amd.processor import CODE, CONTENT, CompressLMProcessor, RequestStatus, SamplingSpec, ServingRequest
from oracle import prefill as op
from oracle import trace as ot


def _proc(C=4, K=2, T=2, policy="rolling", quotas=None):
    codes = list(range(900, 900 + K))
    cfg = CompressLMConfig(replay_tail=0, code_positions="bitrev",
                           enable=True, block_size=C, num_code_tokens=K, retain_tail_kv=T, retain_tail_policy=policy,
                           layer_code_quotas=quotas or (), physical_layer_quotas=bool(quotas))
    cfg.set_code_token_ids(codes)
    proc = CompressLMProcessor(cfg)
    if quotas:
        proc.set_group_quotas(quotas)
    return proc, codes


def run_case(prompt, generated, T=2, policy="rolling", C=4, K=2):
    """The driving loop of scripts/test_compresslm_vllm_state.py:99-214 (block_size 4, two codes, raw prompt); mask
    events are (start, end, num_computed_tokens)."""
    proc, codes = _proc(C, K, T, policy)
    req = ServingRequest("r", prompt, SamplingSpec(max_tokens=len(generated), bad_words_token_ids=[[c] for c in codes]))
    state = proc.prepare_request(req)
    req.compresslm_state = state
    events, gi = [], 0

    def mask_span(_rid, start, end, groups=None):
        assert 0 <= start < end <= req.num_computed_tokens
        events.append((start, end, req.num_computed_tokens))
        return SimpleNamespace(success=True, error_message=None)

    for _ in range(400):
        if req.status != RequestStatus.RUNNING:
            break
        count = proc.limit_num_new_tokens(req, req.num_tokens - req.num_computed_tokens)
        assert count > 0
        start = req.num_computed_tokens
        assert all(state.roles[p] == state.roles[start] for p in range(start, start + count))
        if state.roles[start] == CODE:
            assert count == K
        skip = proc.should_skip_sampling(req, count)
        req.num_computed_tokens += count
        sampled = [] if skip else [generated[gi]]
        gi += 0 if skip else 1
        proc.update_after_step(req, count, sampled, mask_span, max_model_len=256)
    else:
        raise AssertionError("state machine did not terminate")
    assert state.visible_output_token_ids == generated and gi == len(generated)
    for block in state.blocks:
        if block.code_span is None:
            continue
        assert req.all_token_ids[block.code_span[0]:block.code_span[1]] == codes
        assert block.retained_tail_positions == block.content_positions[-T:]
        tail = block.content_positions[-T:]
        assert block.code_excluded_content_span == (tail[0], tail[-1] + 1)
    prompt_pos = {p for b in state.blocks for p in b.prompt_content_positions}
    assert not any(p in prompt_pos for s, e, _ in events for p in range(s, e))
    return req, state, events, proc


def test_config_accepts_the_window_tails_except_with_packed_kv():
    for policy in ("rolling", "sticky"):
        cfg = CompressLMConfig(replay_tail=0, code_positions="bitrev", enable=True, block_size=8, num_code_tokens=4,
                               retain_tail_kv=2, retain_tail_policy=policy)
        assert cfg.code_excluded_tail == 2
        assert cfg.bitrev_code_offsets().max() < 6                          # codes spread over [0, C - T)
        with pytest.raises(ValueError, match="static"):
            CompressLMConfig(replay_tail=0, code_positions="bitrev",
                             enable=True, block_size=8, num_code_tokens=4, retain_tail_kv=2,
                             retain_tail_policy=policy, packed_kv=True, packed_kv_k_max=4)
    assert CompressLMConfig().retain_tail_policy == "rolling"
    with pytest.raises(ValueError, match="retain_tail_kv > 0"):
        CompressLMConfig(replay_tail=0, code_positions="bitrev",
                         enable=True, block_size=8, num_code_tokens=4, retain_tail_policy="sticky")


def test_reference_scenario_rolling():
    """True retention keeps the original pre-code positions, inserts no replay token IDs, and expires one response
    row after each next-block query."""
    req, state, events, _ = run_case([10], [20, 21, 22, 23, 24, 25, 26, 27])
    masks = [(s, e) for s, e, _ in events]
    assert state.blocks[0].retained_tail_positions == [2, 3]
    assert req.all_token_ids[:7] == [10, 20, 21, 22, 900, 901, 23]
    assert (1, 2) in masks and (2, 3) in masks and (3, 4) in masks
    assert state.expired_retained_tail_positions.issuperset({2, 3})
    # row 2 leaves after position 6 (block 1's first content token) ran, row 3 after position 7
    assert (2, 3, 7) in events and (3, 4, 8) in events


def test_reference_scenario_rolling_bulk_limit():
    """A re-prefill that exposes several content tokens at once still schedules one query per expiration."""
    proc, _ = _proc()
    st = SimpleNamespace(roles=[CONTENT] * 8, content_to_expired_replay={}, content_to_expired_retained_tail={2: 0})
    req = SimpleNamespace(compresslm_state=st, num_computed_tokens=2, num_tokens=8)
    assert proc.limit_num_new_tokens(req, proposed=6) == 1
    st.content_to_expired_retained_tail = {3: 0}
    assert proc.limit_num_new_tokens(req, proposed=6) == 2
    sticky, _ = _proc(policy="sticky")
    st.content_to_expired_retained_tail = {}
    assert sticky.limit_num_new_tokens(req, proposed=6) == 6


def test_reference_scenario_sticky_and_its_preemption_replay():
    """Sticky keeps the whole prior response tail through the next block's content and removes it once, right before
    that block's codes; no replay IDs, no rolling expirations. A preemption replays the removal before the existing
    codes are recomputed."""
    req, state, events, proc = run_case([10], list(range(20, 29)), policy="sticky")
    first, second = state.blocks[:2]
    assert first.retained_tail_positions == [2, 3]
    assert not state.content_to_expired_retained_tail and not state.expired_retained_tail_positions
    assert state.expired_sticky_retained_block_ids.issuperset({0})
    boundary = second.content_positions[-1] + 1
    assert events.count((2, 4, boundary)) == 1
    assert events.index((2, 4, boundary)) < events.index((6, 8, second.code_span[1]))
    assert not any(s < 4 and e > 2 and c < boundary for s, e, c in events)
    for tok in [10, *range(20, 28)]:
        assert req.all_token_ids.count(tok) == 1

    proc.reset_for_preemption(state)
    assert not state.expired_sticky_retained_block_ids
    req.num_computed_tokens = 0
    req.status = RequestStatus.RUNNING
    reapplied = []

    def remask(_rid, start, end, groups=None):
        reapplied.append((start, end, req.num_computed_tokens))
        return SimpleNamespace(success=True, error_message=None)

    while req.num_computed_tokens < second.code_span[0]:
        count = proc.limit_num_new_tokens(req, req.num_tokens - req.num_computed_tokens)
        req.num_computed_tokens += count
        proc.update_after_step(req, count, [], remask, max_model_len=256)
    assert (2, 4, boundary) in reapplied
    assert state.expired_sticky_retained_block_ids == {0}


def test_reference_scenario_sticky_tail_straddling_the_prompt():
    """Only the contiguous response suffix of a tail that straddles prompt and response is removed."""
    _, state, events, _ = run_case([30, 31, 32], list(range(40, 49)), policy="sticky")
    first, second = state.blocks[:2]
    assert first.retained_tail_positions == [2, 3]
    boundary = second.content_positions[-1] + 1
    assert events.count((3, 4, boundary)) == 1
    assert not any(s <= 2 < e for s, e, _ in events)


def _drive(policy, prompt_len, gen, C, K, T, quotas, preempt_at=None):
    """Product machine and oracle trace side by side; returns per-step records for the visibility check:
    (kept rows per group before the step, start, n, role)."""
    proc, codes = _proc(C, K, T, policy, quotas)
    req = ServingRequest("r", list(range(100, 100 + prompt_len)),
                         SamplingSpec(max_tokens=gen, bad_words_token_ids=[[c] for c in codes]))
    removed = [[] for _ in quotas]

    def kept(group, upto):
        return [p for p in range(upto) if not any(s <= p < e for s, e in removed[group])]

    def l2p(pos, group=0):
        assert not any(s <= pos < e for s, e in removed[group])
        return pos - sum(e - s for s, e in removed[group] if e <= pos)

    req.logical_to_physical = l2p
    calls = []

    def mask_span(_rid, start, end, groups=None):
        calls.append((start, end, None if groups is None else list(groups)))
        for g in (range(len(quotas)) if groups is None else groups):
            removed[g].append((start, end))
        return SimpleNamespace(success=True, error_message=None)

    state = proc.prepare_request(req)
    req.compresslm_state = state
    tr = ot.RequestTrace(prompt_len, gen, C, K, quotas, retain_tail=T, tail_policy=policy)
    oracle_calls, steps, preempted = [], [], False
    for i in range(4000):
        if req.status != RequestStatus.RUNNING:
            break
        if preempt_at is not None and i == preempt_at:
            proc.reset_for_preemption(state)
            tr.preempt()
            req.num_computed_tokens = 0
            removed = [[] for _ in quotas]
            preempted = True
        count = proc.limit_num_new_tokens(req, req.num_tokens - req.num_computed_tokens)
        assert count == tr.next_chunk()
        start = req.num_computed_tokens
        role = state.roles[start]
        if role == CODE:
            ranges = proc.code_excluded_physical_ranges(req, len(quotas))
            ls, le = proc.code_excluded_logical_range(req)
            for g in range(len(quotas)):
                kg = kept(g, start)
                assert ranges[g] == (kg.index(ls), kg.index(le - 1) + 1)
        steps.append(([kept(g, start) for g in range(len(quotas))], start, count, role))
        skip = proc.should_skip_sampling(req, count)
        req.num_computed_tokens += count
        tr.num_computed_tokens += count
        proc.update_after_step(req, count, [] if skip else [7], mask_span, max_model_len=1 << 20)
        oracle_calls += tr.after_step(count)
        for g in range(len(quotas)):
            assert kept(g, req.num_computed_tokens) == tr.kept_positions(g)
    assert calls == oracle_calls
    assert preempt_at is None or preempted
    return proc, state, tr, steps


CASES = [  # policy, prompt length, generated tokens, C, K, T, group quotas, preempt at step
    ("rolling", 1, 40, 8, 4, 3, (4, 2, 1), None),
    ("rolling", 6, 35, 8, 4, 3, (4, 2), None),
    ("rolling", 13, 30, 8, 4, 3, (4, 1), 23),
    ("rolling", 3, 40, 8, 2, 6, (2,), 31),
    ("sticky", 1, 40, 8, 4, 3, (4, 2, 1), None),
    ("sticky", 10, 35, 8, 4, 3, (4, 2), 19),
    ("sticky", 7, 40, 8, 2, 6, (2, 1), None),
    ("static", 5, 40, 8, 4, 3, (4, 2), 27),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-p{c[1]}-T{c[5]}{'-preempt' if c[7] else ''}" for c in CASES])
def test_product_machine_matches_trace_and_serving_visibility_is_the_training_mask(case):
    """Every query of every step sees exactly its row of the teacher-forced mask: a content query the resident rows
    before the step and its chunk causally; a code query the resident rows minus its block's tail and its block's
    code rows below the group's quota. Logical positions are the mask's sequence indices (C content rows then K code
    rows per block)."""
    policy, prompt_len, gen, C, K, T, quotas, preempt_at = case
    _, state, tr, steps = _drive(policy, prompt_len, gen, C, K, T, quotas, preempt_at)
    assert len(state.compacted_block_ids) >= 3
    N = len(state.blocks)
    per = C + K
    checked = 0
    for g, q in enumerate(quotas):
        mask = op.arith_mask(C, K, N, prompt_len=[prompt_len], head_quota=[q], retain_tail=T,
                             tail_policy=policy)[0, 0]
        for kept, start, n, role in steps:
            before = set(kept[g])
            for p in range(start, start + n):
                if role == CONTENT:
                    got = before | set(range(start, p + 1))
                else:
                    blk = p // per
                    ex = set(range(blk * per + C - T, blk * per + C))
                    got = (before - ex) | set(range(start, start + min(q, K)))
                want = set(np.nonzero(mask[p])[0].tolist())
                assert got == want, (policy, g, p, sorted(got ^ want))
                checked += 1
    assert checked > 50


@pytest.mark.parametrize("policy", ["rolling", "sticky"])
def test_window_tails_leave_the_closed_form_row_count(policy):
    """Resident rows of a group at a content step of block b >= 2 after the window has passed: every closed block
    keeps its raw-prompt rows and q codes; the previous block's response tail is gone (rolling: once T content tokens
    of the block have run; sticky: only after the block's last content token)."""
    C, K, T, quotas = 16, 4, 5, (4, 2)
    tr = ot.RequestTrace(3, 200, C, K, quotas, retain_tail=T, tail_policy=policy)
    seen = 0
    while not tr.finished:
        n = tr.next_chunk()
        tr.num_computed_tokens += n
        tr.after_step(n)
        cur = tr.current_block
        done = [p for p in cur.content_positions if p < tr.num_computed_tokens]
        if cur.block_id < 2 or not done or cur.code_span is not None:
            continue
        for g, q in enumerate(quotas):
            closed = [b for b in tr.blocks if b.block_id in tr.compacted_block_ids]
            want = sum(len(b.prompt_positions) + q for b in closed) + len(done)
            prev = tr.blocks[cur.block_id - 1]
            prev_tail = [p for p in prev.content_positions[-T:] if tr.kind[p] == "response"]
            if policy == "rolling":
                want += sum(1 for i, p in enumerate(prev.content_positions[-T:])
                            if tr.kind[p] == "response" and i >= len(done))
            else:
                want += len(prev_tail)
            assert len(tr.kept_positions(g)) == want
            seen += 1
    assert seen > 50
