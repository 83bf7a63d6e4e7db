"""Pins of oracle.compaction and oracle.trace: brute force over span layouts, pool invariants, the reference's
physical-quota invariants, and the gather-then-scatter execution on identity-tagged caches."""
import random

import numpy as np
import pytest

from oracle import compaction as oc
from oracle import layout as ol
from oracle import trace as ot


def test_span_index_brute_force():
    """scripts/test_compresslm_physical_quotas.py:28-49, restated: 300 random layouts, random.Random(0)."""
    rng = random.Random(0)
    for _ in range(300):
        n = rng.randint(1, 60)
        removed = sorted(rng.sample(range(n), rng.randint(0, n // 2)))
        spans, i = [], 0
        while i < len(removed):
            j = i
            while j + 1 < len(removed) and removed[j + 1] == removed[j] + 1:
                j += 1
            spans.append((removed[i], removed[j] + 1))
            i = j + 1
        index = oc.CompactedSpanIndex(spans)
        active = [p for p in range(n) if p not in removed]
        assert index.total_removed == len(removed)
        assert index.get_active_positions(n) == active
        for phys, logical in enumerate(active):
            assert index.logical_to_physical(logical) == phys
            assert index.physical_to_logical(phys) == logical
            assert index.is_token_active(logical)
        for r in removed:
            assert not index.is_token_active(r)


def test_merge_spans():
    assert oc.merge_spans([(5, 7), (1, 3), (3, 4), (6, 9)]) == [(1, 4), (5, 9)]
    assert oc.merge_spans([]) == []


def test_pool_fifo_reverse_free_and_null_page():
    pool = oc.BlockPool(10)
    assert pool.null_block == 0 and pool.free_queue.order() == list(range(1, 10))
    a = pool.get_new_blocks(3)
    assert a == [1, 2, 3]
    b = pool.get_new_blocks(2)
    pool.free_blocks(reversed(a))
    assert pool.free_queue.order() == [6, 7, 8, 9, 3, 2, 1]
    with pytest.raises(ValueError):
        pool.get_new_blocks(8)
    pool.free_blocks([0])                                 # the null page is never queued
    assert 0 not in pool.free_queue.order()
    assert len(pool.free_queue.order()) + len(b) == 9


def test_truncation_frees_trailing_pages_in_reverse():
    p = oc.Planner(32, 1, 4)
    p.add_request(0)
    p.allocate_slots(0, 20)                               # 5 pages: 1..5
    p.requests[0].num_computed_tokens = 20
    res = p.mask_token_span(0, 2, 15)                     # 13 removed -> 7 active -> 2 pages kept
    assert res.success and res.blocks_freed == 3
    assert p.block_ids(0)[0] == [1, 2]
    assert p.pool.free_queue.order()[-3:] == [5, 4, 3]
    ops, trunc = p.take_step_outputs()
    assert trunc == {0: (2,)}
    # (src, dst) slot pairs (15..19 -> 2..6) in block form with the pre-truncation page list
    assert ops[0][0][0] == [(4, 3, 1, 2), (5, 0, 1, 3), (5, 1, 2, 0), (5, 2, 2, 1), (5, 3, 2, 2)]


def _run_trace_on_oracle(prompt, n_gen, C, K, quotas, block=2):
    """Drive one request through the oracle planner + a tagged numpy cache; yields after every step."""
    tr = ot.RequestTrace(prompt, n_gen, C, K, quotas)
    G = len(quotas)
    pl = oc.Planner(512, G, block)
    pl.add_request(0)
    cache = np.full((512, 2, block, 1, 1), -1, np.int64)     # one tagged "layer" per group shares the tensor
    caches = [[cache] for _ in range(G)]
    steps = 0
    while not tr.finished and steps < 1000:
        n = tr.next_chunk()
        if n == 0:
            break
        assert pl.allocate_slots(0, n) is not None
        start = pl.requests[0].num_computed_tokens
        for g, phys in enumerate(pl.physical_positions(0, np.arange(start, start + n))):
            slots = oc.slot_mapping(pl.block_ids(0)[g], phys, block)
            for s, lp in zip(slots, range(start, start + n)):
                cache[s // block, :, s % block] = lp * 8 + g
        pl.requests[0].num_computed_tokens += n
        tr.num_computed_tokens += n
        for s, e, g in tr.after_step(n):
            assert pl.mask_token_span(0, s, e, g).success
        ops, _ = pl.take_step_outputs()
        oc.execute_kv_copy_operations(ops, caches)
        steps += 1
        yield tr, pl, cache


def test_reference_physical_quota_invariants():
    """scripts/test_compresslm_physical_quotas.py:68-138 restated on the oracle: C=4, K=4, groups (4,2,1,2), prompt
    of 6 tokens, 13 generated. After every step each group's layout keeps exactly codes[:q] of every compacted block
    and no response content, and every kept row holds its own logical token (gather-then-scatter execution)."""
    quotas = (4, 2, 1, 2)
    last = None
    for tr, pl, cache in _run_trace_on_oracle(6, 13, 4, 4, quotas):
        for g, q in enumerate(quotas):
            kept = tr.kept_positions(g)
            idx = pl.requests[0].groups[g]
            assert idx.get_active_positions(tr.num_computed_tokens) == kept
            blocks = pl.block_ids(0)[g]
            assert len(blocks) == -(-len(kept) // 2)
            for phys, lp in enumerate(kept):
                page, off = blocks[phys // 2], phys % 2
                assert cache[page, 0, off, 0, 0] == lp * 8 + g, (g, phys, lp)
            for b in tr.blocks:
                if b.block_id in tr.compacted_block_ids and b.code_span:
                    cs, ce = b.code_span
                    assert [p - cs for p in range(cs, ce) if idx.is_token_active(p)] == list(range(q))
                    assert not any(idx.is_token_active(p) for p in b.response_positions)
        last = (tr, pl)
    tr, pl = last
    n_compacted = len(tr.compacted_block_ids)
    assert n_compacted >= 2
    removed = [pl.requests[0].groups[g].total_removed for g in range(4)]
    for g, q in enumerate(quotas):
        assert removed[g] - removed[0] == n_compacted * (4 - q)


@pytest.mark.parametrize("P,T", [(1, 2), (100, 513), (100, 600), (512, 513), (600, 1300), (1024, 2049),
                                 (300, 2600), (1000, 1025)])
def test_rows_per_layer_matches_simulation(P, T):
    """Simulated request reaching the decode step of content token T-1: seq_len_g = computed - compacted_g + 1
    equals the closed form for every quota group."""
    C, K = 512, 256
    quotas = (256, 64, 128)
    tr = ot.RequestTrace(P, 1 << 30, C, K, quotas)
    removed = [0, 0, 0]
    while True:
        content = sum(1 for k in tr.kind[: tr.num_computed_tokens] if k != "code")
        n = tr.next_chunk()
        if content == T - 1 and tr.roles[tr.num_computed_tokens] == ot.CONTENT:
            break
        tr.num_computed_tokens += n
        for s, e, g in tr.after_step(n):
            for gg in (range(3) if g is None else g):
                removed[gg] += e - s
    for g, q in enumerate(quotas):
        assert tr.num_computed_tokens - removed[g] + 1 == ol.rows_per_layer(T, P, q)
        assert len(tr.kept_positions(g)) + 1 == ol.rows_per_layer(T, P, q)


def test_overlapping_shift_needs_gather_then_scatter():
    """Removing 1 row before a run of 5 moves overlapping slots; the executor must equal the gather-then-scatter
    result (a right-to-left per-op copy would smear the first source row)."""
    cache = np.arange(8 * 2 * 4).reshape(8, 2, 4, 1, 1).astype(np.int64)
    ops = [[[[(1, 1, 1, 0), (1, 2, 1, 1), (1, 3, 1, 2), (2, 0, 1, 3), (2, 1, 2, 0)]]]]
    before = cache.copy()
    oc.execute_kv_copy_operations({0: ops[0]}, [[cache]])
    for s_b, s_o, d_b, d_o in ops[0][0][0]:
        assert np.array_equal(cache[d_b, :, d_o], before[s_b, :, s_o])
    wrong = before.copy()
    for s_b, s_o, d_b, d_o in reversed(ops[0][0][0]):
        wrong[d_b, :, d_o] = wrong[s_b, :, s_o]
    assert not np.array_equal(wrong, cache)


def test_allocate_none_and_error_messages():
    p = oc.Planner(5, 2, 4)
    p.add_request("a")
    assert p.allocate_slots("a", 8) is not None            # 2 pages x 2 groups
    assert p.allocate_slots("a", 9) is None                # needs 2 more, none free
    with pytest.raises(ValueError):
        p.allocate_slots("a", 0)
    p.requests["a"].num_computed_tokens = 8
    assert p.mask_token_span("zz", 0, 1).error_message == "Request zz not found"
    assert p.mask_token_span("a", 3, 3).error_message == "Invalid span: must have 0 <= start < end"
    assert "exceeds computed tokens" in p.mask_token_span("a", 0, 9).error_message
    assert p.mask_token_span("a", 0, 8).error_message == "Cannot compact: all tokens would be removed"
    assert p.mask_token_span("a", 0, 1, [2]).error_message == "KV cache group 2 out of range"
    assert p.mask_token_span("a", 2, 4, [1]).success
    assert "already-removed" in p.mask_token_span("a", 3, 5, [1]).error_message
    assert p.mask_token_span("a", 1, 5, [0]).success      # group 0 still holds [2, 4): one physical span
