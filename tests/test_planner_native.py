"""The native compaction planner (host C++) is bit-exact with the oracle restatement of the reference's scheduler /
KV-manager bookkeeping on seeded multi-request schedules: copy-op batches, truncations, page lists, free-queue
order, span maps and error results. Host logic only (no GPU)."""
import numpy as np
import pytest

from abridgekv_amd.planner import KVPlanner
from oracle import compaction as oc
from tests.planner_harness import compare_state, events_to_array, make_schedule, run_native_step, run_oracle_step

SMALL = dict(C=8, K=4, quotas=(4, 2, 1, 2))          # the reference test's toy geometry (4 groups)
SERVED = dict(C=512, K=256, quotas=(256, 64, 64, 128, 128, 128))


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("geom,block", [(SMALL, 2), (SERVED, 16)])
def test_native_planner_matches_oracle(seed, geom, block):
    C, K, quotas = geom["C"], geom["K"], geom["quotas"]
    n_req = 6 if C == 8 else 4
    steps, _ = make_schedule(seed, n_req, C, K, quotas, max_prompt=3 * C, max_closed=3)
    num_blocks = 4000
    perm = np.random.default_rng(100 + seed).permutation(np.arange(1, num_blocks)).astype(np.int32)
    oracle = oc.Planner(num_blocks, len(quotas), block, free_order=perm)
    native = KVPlanner(num_blocks, len(quotas), block, free_order=perm)
    a_o, a_n = set(), set()
    total_ops = 0
    for events in steps:
        ops_o, tr_o = run_oracle_step(oracle, events, a_o)
        out_n = run_native_step(native, events, a_n)
        assert ops_o == out_n.kv_copy_operations
        assert list(ops_o) == list(out_n.kv_copy_operations), "request order of the op dict differs"
        assert tr_o == out_n.block_table_truncations
        assert list(tr_o) == list(out_n.block_table_truncations)
        total_ops += sum(len(b) for v in ops_o.values() for g in v for b in g)
        compare_state(oracle, native, sorted(a_o))
    assert total_ops > 0


def test_event_batch_api_matches_step_api():
    steps, _ = make_schedule(3, 5, 8, 4, (4, 2, 1, 2), max_prompt=20, max_closed=4)
    perm = np.random.default_rng(0).permutation(np.arange(1, 3000)).astype(np.int32)
    a = KVPlanner(3000, 4, 2, free_order=perm)
    b = KVPlanner(3000, 4, 2, free_order=perm)
    added = set()
    for events in steps:
        run_native_step(a, events, added)
    b.apply_events(events_to_array(steps, 4))
    assert a.free_queue() == b.free_queue()
    for rid in sorted(added):
        assert a.get_blocks(rid) == b.get_blocks(rid)
        assert a.compacted_counts(rid) == b.compacted_counts(rid)


def test_span_errors_match_reference_messages():
    o = oc.Planner(64, 2, 4)
    n = KVPlanner(64, 2, 4)
    for p in (o, n):
        p.add_request(7)
        assert p.allocate_slots(7, 10) is not None
    o.requests[7].num_computed_tokens = 10
    n.set_num_computed_tokens(7, 10)
    cases = [(-1, 3, None), (4, 4, None), (2, 11, None), (0, 2, [5]), (0, 10, None)]
    for s, e, g in cases:
        ro, rn = o.mask_token_span(7, s, e, g), n.mask_token_span(7, s, e, g)
        assert not ro.success and not rn.success
        assert ro.error_message == rn.error_message, (s, e, g)
    assert o.mask_token_span(7, 2, 5).success and n.mask_token_span(7, 2, 5).success
    for s, e in [(4, 6), (1, 3)]:                       # overlaps an already-removed span
        ro, rn = o.mask_token_span(7, s, e), n.mask_token_span(7, s, e)
        assert not ro.success and ro.error_message == rn.error_message
    ro, rn = o.mask_token_span(99, 0, 1), n.mask_token_span(99, 0, 1)
    assert not rn.success and not ro.success


def test_allocation_none_when_pool_exhausted():
    o = oc.Planner(9, 2, 4)
    n = KVPlanner(9, 2, 4)
    for p in (o, n):
        p.add_request(1)
        assert p.allocate_slots(1, 16) is not None        # 4 pages x 2 groups = 8 = all free pages
        assert p.allocate_slots(1, 17) is None
    assert o.pool.free_queue.order() == n.free_queue() == []


def test_free_request_returns_pages_in_reverse_group_order():
    o = oc.Planner(40, 3, 4)
    n = KVPlanner(40, 3, 4)
    for p in (o, n):
        p.add_request(1)
        p.add_request(2)
        p.allocate_slots(1, 9)
        p.allocate_slots(2, 5)
    o.free_request(1)
    n.free(1)
    assert o.pool.free_queue.order() == n.free_queue()


def test_compaction_workload_64_sequences_matches_oracle():
    """The compaction workload at its benched size: 64 sequences with seeded prompts and 0-3 earlier closed blocks,
    a seeded fragmented free list, the served geometry (C=512, K=256, six Qwen3-4B quota groups). The whole replayed
    history and then the compaction step itself go through the oracle planner; copy-op batches (per request, per
    group, in order), truncations, free-queue order, page lists, compacted counts, span maps and the page tables the
    worker would hold must all be identical."""
    from abridgekv_amd import workloads
    from tests.planner_harness import apply_events_oracle

    st = workloads.build_compaction_state(64, seed=0)
    G = len(st.groups)
    oracle = oc.Planner(st.num_pages, G, 16, free_order=st.free_order)
    apply_events_oracle(oracle, st.history)
    oracle.take_step_outputs()
    rids = list(range(64))
    compare_state(oracle, st.planner, rids)
    apply_events_oracle(oracle, st.pending)
    ops_o, tr_o = oracle.take_step_outputs()
    st.planner.apply_events(st.pending)
    out = st.planner.take_step_outputs()
    assert ops_o == out.kv_copy_operations
    assert list(ops_o) == list(out.kv_copy_operations)
    assert tr_o == out.block_table_truncations
    assert sum(len(b) for v in ops_o.values() for g in v for b in g) > 64 * 256
    compare_state(oracle, st.planner, rids)
    for g in range(G):
        W = max(len(oracle.block_ids(r)[g]) for r in rids)
        ref = np.zeros((64, W), np.int32)
        for r in rids:
            ids = oracle.block_ids(r)[g]
            ref[r, :len(ids)] = ids
        assert np.array_equal(st.planner.fill_block_table(rids, g, W), ref), f"group {g}"


def test_fused_only_planner_keeps_the_bookkeeping_and_the_fused_moves():
    """op_rows=False skips the reference-format op batches only: on the 64-sequence compaction step and on served
    multi-step schedules, page lists, spans, truncations, the free queue and the fused moves equal those of the planner
    that builds the op batches, and no op rows are emitted."""
    from abridgekv_amd import workloads

    a = workloads.build_compaction_state(64, seed=0)
    b = workloads.build_compaction_state(64, seed=0, op_rows=False)
    ops_a, tr_a, fu_a = a.compact(as_arrays=True)
    ops_b, tr_b, fu_b = b.compact(as_arrays=True)
    assert len(ops_a) > 64 * 256 and len(ops_b) == 0
    assert np.array_equal(tr_a, tr_b) and np.array_equal(fu_a, fu_b)
    assert a.planner.free_queue() == b.planner.free_queue()
    for r in range(64):
        assert a.planner.get_blocks(r) == b.planner.get_blocks(r)
        assert a.planner.compacted_counts(r) == b.planner.compacted_counts(r)
    quotas = SERVED["quotas"]
    for seed in range(3):
        steps, _ = make_schedule(seed, 4, SERVED["C"], SERVED["K"], quotas, max_prompt=3 * SERVED["C"], max_closed=3)
        perm = np.random.default_rng(100 + seed).permutation(np.arange(1, 4000)).astype(np.int32)
        full = KVPlanner(4000, len(quotas), 16, free_order=perm)
        fused = KVPlanner(4000, len(quotas), 16, free_order=perm, op_rows=False)
        seen_a, seen_b = set(), set()
        for events in steps:
            out_a = run_native_step(full, events, seen_a)
            out_b = run_native_step(fused, events, seen_b)
            assert out_b.kv_copy_operations == {}
            assert out_a.block_table_truncations == out_b.block_table_truncations
            assert np.array_equal(out_a.fused_moves, out_b.fused_moves)
        assert full.free_queue() == fused.free_queue()
        for r in sorted(seen_a):
            assert full.get_blocks(r) == fused.get_blocks(r)
            for g in range(len(quotas)):
                assert full.group_compacted_spans(r, g) == fused.group_compacted_spans(r, g)
