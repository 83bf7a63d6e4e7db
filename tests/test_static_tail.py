"""The static retained tail (retain_tail_kv = T, retain_tail_policy="static") on the CPU: configuration, the state
machine's removal spans and code-step exclusion ranges, against the reference's own static-tail scenarios
(scripts/test_compresslm_vllm_state.py:302-351) and the oracle trace."""
from types import SimpleNamespace

import pytest

from abridgekv_amd.config import CompressLMConfig
from abridgekv_amd.processor import CODE, CompressLMProcessor, RequestStatus, SamplingSpec, ServingRequest
from oracle import trace as ot


def run_case(prompt, generated, T=2, packed=False, quotas=None, C=4, K=2):
    """The driving loop of scripts/test_compresslm_vllm_state.py:99-214 (block_size 4, two codes, raw prompt):
    returns (request, state, masks, pack events)."""
    codes = list(range(900, 900 + K))
    cfg = CompressLMConfig(replay_tail=0, code_positions="bitrev",
                           enable=True, block_size=C, num_code_tokens=K, retain_tail_kv=T, retain_tail_policy="static",
                           packed_kv=packed, packed_kv_k_max=K if packed else 2048,
                           layer_code_quotas=quotas or (), physical_layer_quotas=bool(quotas))
    cfg.set_code_token_ids(codes)
    proc = CompressLMProcessor(cfg)
    if quotas:
        proc.set_group_quotas(quotas)
    req = ServingRequest("r", prompt, SamplingSpec(max_tokens=len(generated), bad_words_token_ids=[[c] for c in codes]))
    state = proc.prepare_request(req)
    req.compresslm_state = state
    masks, packs, gi = [], [], 0

    def mask_span(_rid, start, end, groups=None):
        assert 0 <= start < end <= req.num_computed_tokens
        masks.append((start, end) if groups is None else (start, end, tuple(groups)))
        return SimpleNamespace(success=True, error_message=None)

    for _ in range(400):
        if req.status != RequestStatus.RUNNING:
            break
        count = proc.limit_num_new_tokens(req, req.num_tokens - req.num_computed_tokens)
        assert count > 0
        if state.roles[req.num_computed_tokens] == CODE:
            assert count == K
        skip = proc.should_skip_sampling(req, count)
        req.num_computed_tokens += count
        sampled = [] if skip else [generated[gi]]
        gi += 0 if skip else 1
        proc.update_after_step(req, count, sampled, mask_span, max_model_len=256,
                               pack_code_span=(lambda _r, s, e: packs.append((s, e))) if packed else None)
    else:
        raise AssertionError("state machine did not terminate")
    assert state.visible_output_token_ids == generated
    for block in state.blocks:
        if block.code_span is None:
            continue
        assert block.retained_tail_positions == block.content_positions[-T:]
        tail = block.content_positions[-T:]
        assert block.code_excluded_content_span == (tail[0], tail[-1] + 1)
    prompt_pos = {p for b in state.blocks for p in b.prompt_content_positions}
    assert not any(p in prompt_pos for m in masks for p in range(m[0], m[1]))
    return req, state, masks, packs


def test_config_static_tail():
    cfg = CompressLMConfig(replay_tail=0, code_positions="bitrev",
                           enable=True, block_size=8, num_code_tokens=4, retain_tail_kv=2, retain_tail_policy="static",
                           packed_kv=True, packed_kv_k_max=4)
    assert cfg.code_excluded_tail == 2
    offs = cfg.bitrev_code_offsets().tolist()
    assert max(offs) < 6 and len(set(offs)) == 4 and offs[0] == 0, offs       # grid over [0, C - T) = [0, 6)
    assert CompressLMConfig(replay_tail=0, code_positions="bitrev",
                            enable=True, block_size=8, num_code_tokens=4).code_excluded_tail == 0
    with pytest.raises(ValueError, match="retain_tail_policy"):
        CompressLMConfig(retain_tail_policy="invalid")
    with pytest.raises(ValueError, match="retain_tail_kv > 0"):
        CompressLMConfig(replay_tail=0, code_positions="bitrev",
                         enable=True, block_size=8, num_code_tokens=4, retain_tail_policy="sticky")
    for policy in ("rolling", "sticky"):                                     # window tails: not with packed KV
        with pytest.raises(ValueError, match="static"):
            CompressLMConfig(replay_tail=0, code_positions="bitrev",
                             enable=True, block_size=8, num_code_tokens=4, retain_tail_kv=2, retain_tail_policy=policy,
                             packed_kv=True, packed_kv_k_max=4)
    with pytest.raises(ValueError, match="block_size"):
        CompressLMConfig(replay_tail=0, code_positions="bitrev",
                         enable=True, block_size=8, num_code_tokens=4, retain_tail_kv=8, retain_tail_policy="static")
    with pytest.raises(ValueError, match="span"):
        CompressLMConfig(replay_tail=0, code_positions="bitrev",
                         enable=True, block_size=8, num_code_tokens=4, retain_tail_kv=6, retain_tail_policy="static")
    # export keeps the tail fields (compresslm_config.json)
    meta = cfg.to_metadata()
    assert meta["retain_tail_kv"] == 2 and meta["retain_tail_policy"] == "static"


def test_reference_scenario_static_dense():
    """STATIC without packed KV: only the response prefix is removed; codes and tails stay resident."""
    _, state, masks, _ = run_case([10], [20, 21, 22, 23, 24, 25, 26, 27])
    assert (1, 2) in masks and all(m[0] >= 1 for m in masks)
    assert (4, 6) not in masks and (2, 4) not in masks
    b0 = state.blocks[0]
    assert b0.retained_tail_positions == [2, 3] and b0.code_span == (4, 6) and b0.code_excluded_content_span == (2, 4)
    assert masks[0] == (1, 2)
    _, state, masks, _ = run_case([10], list(range(20, 32)))                # a second block closes as well
    b1 = state.blocks[1]
    assert masks == [(1, 2), (b1.response_content_positions[0], b1.retained_tail_positions[0])]


def test_reference_scenario_static_packed():
    """STATIC + packed KV: the block's final T content rows stay resident; the summarized response content and the
    code span are removed as two separate spans around them, after the codes are archived."""
    _, state, masks, packs = run_case([10], [20, 21, 22, 23, 24, 25, 26, 27, 28, 29], packed=True)
    b0, b1 = state.blocks[0], state.blocks[1]
    assert b0.retained_tail_positions == [2, 3] and b0.code_span == (4, 6)
    assert packs[0] == b0.code_span and packs[1] == b1.code_span
    assert (1, 2) in masks and (4, 6) in masks
    assert (2, 3) not in masks and (3, 4) not in masks and (2, 4) not in masks
    assert (b1.response_content_positions[0], b1.retained_tail_positions[0]) in masks
    assert b1.code_span in masks
    assert b0.code_excluded_content_span == (2, 4)
    assert b1.code_excluded_content_span == (b1.retained_tail_positions[0], b1.retained_tail_positions[-1] + 1)


@pytest.mark.parametrize("prompt_len,gen", [(1, 30), (6, 25), (13, 17)])
def test_physical_quotas_with_static_tail_match_oracle_trace(prompt_len, gen):
    """Physical per-layer quotas with a static tail: the product machine issues the oracle trace's calls (response
    prefix before the tail in every group, then code slots [q, K) per quota), and each code step's physical
    exclusion range in every group is where the block's tail lies in that group's brute-force kept stream."""
    quotas, C, K, T = (4, 2, 1, 2), 8, 4, 3
    codes = list(range(900, 900 + K))
    cfg = CompressLMConfig(replay_tail=0, code_positions="bitrev",
                           enable=True, block_size=C, num_code_tokens=K, retain_tail_kv=T, retain_tail_policy="static",
                           layer_code_quotas=quotas, physical_layer_quotas=True)
    cfg.set_code_token_ids(codes)
    proc = CompressLMProcessor(cfg)
    proc.set_group_quotas(quotas)
    req = ServingRequest("r", list(range(100, 100 + prompt_len)),
                         SamplingSpec(max_tokens=gen, bad_words_token_ids=[[c] for c in codes]))
    removed = [[] for _ in quotas]

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
    tr = ot.RequestTrace(prompt_len, gen, C, K, quotas, retain_tail=T)
    oracle_calls, gi, n_code_steps = [], 0, 0
    for _ in range(800):
        if req.status != RequestStatus.RUNNING:
            break
        count = proc.limit_num_new_tokens(req, req.num_tokens - req.num_computed_tokens)
        assert count == tr.next_chunk()
        if state.roles[req.num_computed_tokens] == CODE:
            n_code_steps += 1
            ranges = proc.code_excluded_physical_ranges(req, len(quotas))
            ls, le = proc.code_excluded_logical_range(req)
            for g in range(len(quotas)):
                kept = [p for p in range(req.num_computed_tokens) if not any(s <= p < e for s, e in removed[g])]
                assert ranges[g] == (kept.index(ls), kept.index(le - 1) + 1)
        skip = proc.should_skip_sampling(req, count)
        req.num_computed_tokens += count
        tr.num_computed_tokens += count
        sampled = [] if skip else [7]
        gi += 0 if skip else 1
        proc.update_after_step(req, count, sampled, mask_span, max_model_len=1 << 20)
        oracle_calls += tr.after_step(count)
    assert n_code_steps >= 2 and calls == oracle_calls
    for g in range(len(quotas)):                                            # the oracle's kept stream, brute force
        kept = [p for p in range(req.num_computed_tokens) if not any(s <= p < e for s, e in removed[g])]
        assert kept == tr.kept_positions(g)
    for b in state.blocks:                                                  # tails survive in every group
        if b.block_id in state.compacted_block_ids:
            for g in range(len(quotas)):
                assert all(not any(s <= p < e for s, e in removed[g]) for p in b.retained_tail_positions)


def test_oracle_trace_static_tail_rows_closed_form():
    """Rows a group keeps with a static tail: every closed block keeps its prompt content, its last T content rows
    and q codes; the open block its content so far (the closed form of oracle.layout.rows_per_layer plus T per
    closed response block)."""
    C, K, T = 16, 4, 5
    quotas = (4, 2)
    for prompt_len in (3, 16, 21, 40):
        tr = ot.RequestTrace(prompt_len, 200, C, K, quotas, retain_tail=T)
        steps = 0
        while not tr.finished and steps < 2000:
            n = tr.next_chunk()
            tr.num_computed_tokens += n
            tr.after_step(n)
            steps += 1
            if tr.roles[tr.num_computed_tokens - 1] == ot.CONTENT and not any(
                    b.code_span and b.code_span[0] <= tr.num_computed_tokens - 1 < b.code_span[1] for b in tr.blocks):
                for g, q in enumerate(quotas):
                    closed = [b for b in tr.blocks if b.block_id in tr.compacted_block_ids]
                    want = 0
                    for b in closed:
                        tail = set(b.content_positions[-T:])
                        want += len(b.prompt_positions) + sum(1 for p in b.response_positions if p in tail) + q
                    want += len([p for p in tr.current_block.content_positions if p < tr.num_computed_tokens])
                    assert len(tr.kept_positions(g)) == want
        assert len(tr.compacted_block_ids) >= 3
