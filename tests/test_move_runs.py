"""The planner's run descriptors (abkv_planner_take_move_runs) on the CPU: expanded with the closed-form row map the
device kernel uses (restated here in numpy), they give exactly the move lists the planner writes row by row
(abkv_planner_take_moves_packed) -- same index, same int32 elements -- on the 64-sequence compaction step and on
multi-step served schedules, with the same truncation rows and free queue."""
import numpy as np
import pytest

from abridgekv_amd import workloads
from abridgekv_amd.planner import KVPlanner
from tests.planner_harness import make_schedule, run_events

PAGE = 16
F, M = KVPlanner.RUN_FIELDS, 8


def expand(buf, layout, n_elems, G, shift=4):
    """Host restatement of moves_expand_kernel: final row i came from f(i) = i + c[J(i)]; ordered ops are the rows of
    A = [t_star, a_end) and of B = f(A), ranked by |A before i| + |B before i| - |A n B before i|."""
    runs_at, n_runs, pages_at, groups_at = layout
    out = np.full(n_elems, -7, np.int32)                   # any element left unwritten shows up
    gr = buf[groups_at: groups_at + 4 * G].reshape(G, 4)
    n_pages = groups_at - pages_at                          # the kernel's n_pages: entries of the page section
    for g in range(G):
        assert gr[g, 0] >= 0 and gr[g, 1] >= 0                # the kernel skips a group row that fails this
        out[gr[g, 0]] = 0
        out[gr[g, 0] + 1 + gr[g, 1]: gr[g, 2]] = 0
    pages = buf[pages_at:]
    for rec in buf[runs_at: runs_at + F * n_runs].reshape(n_runs, F):
        n, lo_w, pat, ord_at, free_at, n_ch, n_free, seg_at, seg_val, m, t_star, a_end, win_n = map(int, rec[:13])
        assert 0 <= pat and 0 <= win_n and pat + win_n <= n_pages     # the kernel skips a record that fails this
        tau = [int(x) for x in rec[14:14 + m]]
        c = [int(x) for x in rec[14 + M:14 + M + m]]
        if seg_at >= 0:
            out[seg_at] = seg_val

        def f(x):
            add = 0
            for j in range(m):
                add = c[j] if x >= tau[j] else add
            return x + add

        def inv(y):
            for j in range(m + 1):
                x = max(0 if j == 0 else tau[j - 1], y - (0 if j == 0 else c[j - 1]))
                if j == m or x < tau[j]:
                    return x

        for i in range(t_star, n):
            src, dst = lo_w + f(i), lo_w + i
            gi = inv(i)
            ordered = i < a_end or (t_star <= gi < a_end and f(gi) == i)
            rank = (min(i - t_star, a_end - t_star) + max(0, min(a_end, gi) - t_star)
                    - max(0, min(a_end, inv(min(i, a_end))) - t_star))
            if ordered:
                assert 0 <= rank < n_ch
                pos = ord_at + 4 * rank
            else:
                assert 0 <= i - t_star - rank < n_free
                pos = free_at + 4 * (i - t_star - rank)
            assert 0 <= src and 0 <= dst and src >> shift < win_n and dst >> shift < win_n
            out[pos:pos + 4] = (pages[pat + (src >> shift)], src & (PAGE - 1), pages[pat + (dst >> shift)],
                                dst & (PAGE - 1))
    return out


def test_runs_expand_to_the_packed_lists_on_the_64_sequence_step():
    a = workloads.build_compaction_state(64, seed=0, op_rows=False)
    b = workloads.build_compaction_state(64, seed=0, op_rows=False)
    a.planner.apply_events(a.pending)
    b.planner.apply_events(b.pending)
    tr_a, buf_a, parts_a = a.planner.take_step_moves()
    tr_b, desc, layout, parts_b, n_elems = b.planner.take_step_move_runs()
    assert parts_a == parts_b and np.array_equal(tr_a, tr_b) and n_elems == buf_a.size
    assert desc.size * 5 < buf_a.size                      # the descriptors are a fraction of the lists
    assert np.array_equal(expand(desc, layout, n_elems, b.planner.num_groups), buf_a)
    assert a.planner.free_queue() == b.planner.free_queue()
    for g in range(a.planner.num_groups):
        assert a.planner.fill_block_table(list(range(64)), g, 2100).tolist() == \
            b.planner.fill_block_table(list(range(64)), g, 2100).tolist()


@pytest.mark.parametrize("seed", range(4))
def test_runs_expand_to_the_packed_lists_on_served_schedules(seed):
    quotas = (256, 64, 64, 128, 128, 128)
    steps, _ = make_schedule(seed, 4, 512, 256, quotas, max_prompt=3 * 512, max_closed=3)
    perm = np.random.default_rng(100 + seed).permutation(np.arange(1, 4000)).astype(np.int32)
    pa = KVPlanner(4000, len(quotas), PAGE, free_order=perm, op_rows=False)
    pb = KVPlanner(4000, len(quotas), PAGE, free_order=perm, op_rows=False)
    seen_a, seen_b = set(), set()
    checked = 0
    for events in steps:
        run_events(pa, events, seen_a)
        run_events(pb, events, seen_b)
        tr_a, buf_a, parts_a = pa.take_step_moves()
        tr_b, desc, layout, parts_b, n_elems = pb.take_step_move_runs()
        assert parts_a == parts_b and np.array_equal(tr_a, tr_b)
        if parts_a:
            assert np.array_equal(expand(desc, layout, n_elems, len(quotas)), buf_a)
            checked += 1
        assert pa.free_queue() == pb.free_queue()
    assert checked >= 3


def test_runs_need_a_large_enough_buffer():
    b = workloads.build_compaction_state(8, seed=0, op_rows=False)
    b.planner.apply_events(b.pending)
    with pytest.raises(ValueError, match="at least"):
        b.planner.take_step_move_runs(np.zeros(8, np.int32))
    _, desc, layout, parts, n_elems = b.planner.take_step_move_runs()   # the step was not cleared by the failure
    assert parts and n_elems > 0


@pytest.mark.parametrize("n_removals", [8, 9])
def test_many_removals_in_one_step(n_removals):
    """Up to eight span removals of one request and group in one step expand to the packed lists; a ninth is refused
    with the planner's message (the step is left pending, so the host-written lists can still be taken)."""
    pa, pb = (KVPlanner(200, 1, PAGE, op_rows=False) for _ in range(2))
    for p in (pa, pb):
        p.add_request(7)
        assert p.allocate_slots(7, 1000) is not None
        p.set_num_computed_tokens(7, 1000)
        for k in range(n_removals):                         # disjoint logical spans in a scrambled order
            s = 40 + 100 * ((5 * k) % n_removals)
            assert p.mask_token_span(7, s, s + 10 + k).success
    tr_a, buf_a, parts_a = pa.take_step_moves()
    if n_removals <= 8:
        tr_b, desc, layout, parts_b, n_elems = pb.take_step_move_runs()
        assert parts_a == parts_b and np.array_equal(tr_a, tr_b)
        assert np.array_equal(expand(desc, layout, n_elems, 1), buf_a)
    else:
        with pytest.raises(RuntimeError, match="more than 8 span removals"):
            pb.take_step_move_runs()
        tr_b, buf_b, parts_b = pb.take_step_moves()
        assert parts_a == parts_b and np.array_equal(buf_a, buf_b)


@pytest.mark.parametrize("n_removals", [8, 9])
def test_step_move_lists_fall_back_to_host_lists(n_removals):
    """worker.take_step_move_lists: run descriptors while the planner accepts them; past eight removals of one request
    and group in a step, the host-written lists of the still-pending step -- the same lists either way."""
    from abridgekv_amd.worker import take_step_move_lists
    pa, pb = (KVPlanner(200, 1, PAGE, op_rows=False) for _ in range(2))
    for p in (pa, pb):
        p.add_request(7)
        assert p.allocate_slots(7, 1000) is not None
        p.set_num_computed_tokens(7, 1000)
        for k in range(n_removals):
            s = 40 + 100 * ((7 * k) % n_removals)
            assert p.mask_token_span(7, s, s + 10 + k).success
    _, want, parts_a = pa.take_step_moves()
    kind, buf, layout, parts_b, n_elems = take_step_move_lists(pb)
    assert kind == ("runs" if n_removals <= 8 else "packed") and parts_a == parts_b
    got = expand(buf, layout, n_elems, 1) if kind == "runs" else buf
    assert np.array_equal(got, want) and n_elems == want.size
    assert pb.take_step_moves()[2] == []                   # the step was taken


@pytest.mark.parametrize("order", ["descending", "scrambled"])
def test_moves_when_a_later_removal_of_the_step_starts_lower(order):
    """The planner keeps only the part of a step's page list at or after the step's lowest removal, and extends it
    downward when a later removal starts below the earlier ones: the fused moves (gather-then-scatter) must leave every
    kept row holding the row id of its logical position's slot before the step, and the same ids as the reference's
    ordered op batches applied one after the other (oracle executor); the host-written lists and the expanded run
    descriptors must agree. Removals in descending and scrambled order over two groups (some in one group only), with
    pages freed by the truncations."""
    from oracle import compaction as oc

    spans = [(700, 730, None), (420, 450, [1]), (90, 100, None), (300, 305, [0]), (20, 40, None)]
    if order == "scrambled":
        spans = [spans[i] for i in (3, 0, 4, 1, 2)]
    G, pages = 2, 400
    planners = [KVPlanner(pages, G, PAGE, free_order=np.arange(1, pages, dtype=np.int32)) for _ in range(3)]
    for p in planners:
        p.add_request(7)
        assert p.allocate_slots(7, 1000) is not None
        p.set_num_computed_tokens(7, 1000)
    before = planners[0].get_blocks(7)
    for p in planners:
        for s, e, groups in spans:
            assert p.mask_token_span(7, s, e, groups).success
    pa, pb, pc = planners
    out = pa.take_step_outputs()
    _, buf_b, parts_b = pb.take_step_moves()
    _, desc, layout, parts_c, n_elems = pc.take_step_move_runs()
    assert parts_b == parts_c and np.array_equal(expand(desc, layout, n_elems, G), buf_b)
    fused = np.asarray(out.fused_moves, np.int64)
    assert sum(n for _, _, n, _, _, _ in parts_b) == len(fused)
    image = np.arange(pages * PAGE, dtype=np.int64).reshape(pages, PAGE)
    for g in range(G):
        rows = fused[fused[:, 1] == g]
        mine = image.copy()
        mine[rows[:, 4], rows[:, 5]] = image[rows[:, 2], rows[:, 3]]          # gather, then scatter
        ref = np.stack([image, image], axis=1).copy()
        oc.execute_kv_copy_operations({r: [b if i == g else [] for i, b in enumerate(v)]
                                       for r, v in out.kv_copy_operations.items()},
                                      [[ref] if i == g else [] for i in range(G)])
        removed = {x for s, e, gs in spans if gs is None or g in gs for x in range(s, e)}
        kept = np.array([x for x in range(1000) if x not in removed])
        active = pa.num_computed_tokens(7) - pa.compacted_counts(7)[g]
        assert len(kept) == active
        slots = oc.slot_mapping(pa.get_blocks(7)[g], np.arange(active))
        want = oc.slot_mapping(before[g], kept)                                 # each kept row's slot before the step
        assert np.array_equal(mine[slots // PAGE, slots % PAGE], want), g
        assert np.array_equal(ref[slots // PAGE, 0, slots % PAGE], want), g
