"""Host packing of a planner step's fused moves into device move lists (abkv_moves_pack), without a GPU.

Exactness is checked on a CPU model of the mixed launch (abkv_kv_move_mixed): every workgroup's load phase and store
phase are separate events, and the events of all workgroups are interleaved at random (each workgroup's own events
in order). Ordered segments are walked 64 ops per chunk, independent ops 4 per workgroup, as the kernel does. The
result must equal gather-then-scatter of the step's fused rows (the reference executor's semantics,
gpu_model_runner.py:1194-1224) for every interleaving; a negative control shows that the model catches a run with a
dependency that is wrongly treated as independent.
"""
import numpy as np
import pytest

from abridgekv_amd import worker, workloads
from abridgekv_amd.planner import KVPlanner
from tests.planner_harness import make_schedule, run_native_step

PAGE = 16


def gather_then_scatter(cache, rows):
    out = cache.copy()
    out[rows[:, 4], rows[:, 5]] = cache[rows[:, 2], rows[:, 3]]
    return out


def phases(ops_g, offs, n_free, chunk=64, free_rows=4):
    """Workgroups of the mixed launch, each a list of op-index chunks: (load all, then store all) per chunk."""
    wgs = []
    for s in range(len(offs) - 1):
        wgs.append([np.arange(a, min(a + chunk, offs[s + 1])) for a in range(offs[s], offs[s + 1], chunk)])
    f0 = offs[-1]
    for a in range(f0, f0 + n_free, free_rows):
        wgs.append([np.arange(a, min(a + free_rows, f0 + n_free))])
    return wgs


def run_model(cache, ops_g, wgs, rng):
    """Random interleaving of the workgroups' load and store events."""
    c = cache.copy()
    state = [(0, None) for _ in wgs]                       # (chunk index, loaded values or None)
    live = list(range(len(wgs)))
    while live:
        k = int(rng.integers(len(live)))
        w = live[k]
        ci, vals = state[w]
        idx = wgs[w][ci]
        if vals is None:
            state[w] = (ci, c[ops_g[idx, 0], ops_g[idx, 1]].copy())
        else:
            c[ops_g[idx, 2], ops_g[idx, 3]] = vals
            state[w] = (ci + 1, None)
            if ci + 1 == len(wgs[w]):
                live.pop(k)
    return c


def unpack(buf, parts):
    out = {}
    for gid, o, n, so, ns, nf in parts:
        out[gid] = (buf[o: o + 4 * n].reshape(-1, 4), buf[so: so + ns + 1], nf)
    return out


@pytest.fixture(scope="module")
def compaction_step():
    st = workloads.build_compaction_state(64, seed=0)
    _, _, fused = st.compact(as_arrays=True)
    return st, np.asarray(fused, dtype=np.int64).copy()


def on_dependency(run):
    """Indices of a run's ops that lie on a dependency: op j writes the slot op i reads (both are on it)."""
    src = {(b, o): i for i, (b, o, _, _) in enumerate(run)}
    on = set()
    for j, (_, _, b, o) in enumerate(run):
        if (b, o) in src:
            on |= {src[(b, o)], j}
    return on


def test_pack_layout_dependent_ops_ordered_then_independent(compaction_step):
    st, fm = compaction_step
    buf, parts = worker.pack_fused_moves(fm, st.num_pages)
    got = unpack(buf, parts)
    assert sorted(got) == list(range(len(st.groups)))
    n_seg_total = n_free_total = 0
    for gid, (ops_g, offs, nf) in got.items():
        rows = fm[fm[:, 1] == gid]
        assert ops_g.shape[0] == rows.shape[0]
        assert offs[0] == 0 and offs[-1] + nf == rows.shape[0]
        runs = {}
        for r in rows:
            runs.setdefault(int(r[0]), []).append(tuple(int(x) for x in r[2:6]))
        want_segs, want_free = [], []
        for run in runs.values():                          # emission order of the runs
            on = on_dependency(run)
            if on:
                want_segs.append([run[i] for i in sorted(on)])
            want_free += [run[i] for i in range(len(run)) if i not in on]
        segs = [[tuple(int(x) for x in op) for op in ops_g[offs[s]: offs[s + 1]]] for s in range(len(offs) - 1)]
        assert segs == want_segs
        assert [tuple(int(x) for x in op) for op in ops_g[offs[-1]:]] == want_free
        n_seg_total += len(segs)
        n_free_total += nf
    assert n_seg_total > 0 and n_free_total > 0            # both kinds are exercised


def test_mixed_launch_model_equals_gather_then_scatter(compaction_step):
    st, fm = compaction_step
    buf, parts = worker.pack_fused_moves(fm, st.num_pages)
    rng = np.random.default_rng(0)
    cache = rng.integers(0, 1 << 30, size=(st.num_pages, PAGE))
    for gid, (ops_g, offs, nf) in unpack(buf, parts).items():
        ref = gather_then_scatter(cache, fm[fm[:, 1] == gid])
        wgs = phases(ops_g, offs, nf)
        for trial in range(2):
            assert np.array_equal(run_model(cache, ops_g, wgs, rng), ref), (gid, trial)


def test_model_catches_dependent_ops_treated_as_independent(compaction_step):
    """Negative control: treat every op of a group as independent, 4 ops per workgroup; some interleaving of the
    model then reads a slot after another workgroup overwrote it."""
    st, fm = compaction_step
    buf, parts = worker.pack_fused_moves(fm, st.num_pages)
    gid, (ops_g, offs, nf) = next((g, v) for g, v in unpack(buf, parts).items() if len(v[1]) > 1)
    bad_offs = np.array([0], np.int64)                     # no ordered segments: everything independent
    wgs = phases(ops_g, bad_offs, ops_g.shape[0])
    rng = np.random.default_rng(1)
    cache = rng.integers(0, 1 << 30, size=(st.num_pages, PAGE))
    ref = gather_then_scatter(cache, fm[fm[:, 1] == gid])
    assert any(not np.array_equal(run_model(cache, ops_g, wgs, rng), ref) for _ in range(5))


@pytest.mark.parametrize("seed", range(4))
def test_pack_over_served_schedules(seed):
    """Multi-step schedules at the served geometry (C=512, K=256, six quota groups): every step's packed moves, run
    through the launch model, equal gather-then-scatter of that step's fused rows."""
    quotas = (256, 64, 64, 128, 128, 128)
    steps, _ = make_schedule(seed, 4, 512, 256, quotas, max_prompt=3 * 512, max_closed=3)
    perm = np.random.default_rng(100 + seed).permutation(np.arange(1, 4000)).astype(np.int32)
    planner = KVPlanner(4000, len(quotas), PAGE, free_order=perm)
    added = set()
    rng = np.random.default_rng(seed)
    cache = rng.integers(0, 1 << 30, size=(4000, PAGE))
    n_checked = 0
    for events in steps:
        out = run_native_step(planner, events, added)
        fm = np.asarray(out.fused_moves, dtype=np.int64)
        if fm.size == 0:
            continue
        buf, parts = worker.pack_fused_moves(fm, 4000, num_groups=len(quotas))
        for gid, (ops_g, offs, nf) in unpack(buf, parts).items():
            ref = gather_then_scatter(cache, fm[fm[:, 1] == gid])
            assert np.array_equal(run_model(cache, ops_g, phases(ops_g, offs, nf), rng), ref)
            n_checked += 1
    assert n_checked > 0


def test_pack_rejects_inputs_the_launch_cannot_run():
    ok = np.array([[1, 0, 5, 3, 5, 0], [1, 0, 5, 4, 5, 1]], np.int64)
    worker.pack_fused_moves(ok, 16)
    raw = np.array([[1, 0, 5, 1, 5, 0], [1, 0, 5, 2, 5, 1], [1, 0, 5, 0, 5, 2]], np.int64)   # op 2 reads a slot op 0 wrote
    with pytest.raises(ValueError):
        worker.pack_fused_moves(raw, 16)
    split_run = np.array([[1, 0, 5, 3, 5, 0], [2, 0, 6, 3, 6, 0], [1, 0, 5, 4, 5, 1]], np.int64)
    with pytest.raises(ValueError):
        worker.pack_fused_moves(split_run, 16)
    with pytest.raises(ValueError):
        worker.pack_fused_moves(ok, 16, num_groups=0)
    twice = np.array([[1, 0, 5, 3, 5, 0], [1, 0, 5, 3, 5, 1]], np.int64)                    # one slot read twice
    with pytest.raises(ValueError):
        worker.pack_fused_moves(twice, 16)


@pytest.mark.parametrize("op_rows", [True, False])
def test_planner_writes_the_same_move_lists_directly(op_rows):
    """KVPlanner.take_step_moves (the planner writing the packed lists itself, dependencies from physical positions)
    equals take_step_outputs followed by pack_fused_moves, element for element, with the same truncation rows: on the
    64-sequence step and on served multi-step schedules."""
    a = workloads.build_compaction_state(64, seed=0, op_rows=op_rows)
    b = workloads.build_compaction_state(64, seed=0, op_rows=op_rows)
    _, tr_a, fu_a = a.compact(as_arrays=True)
    buf_a, parts_a = worker.pack_fused_moves(fu_a, a.num_pages)
    b.planner.apply_events(b.pending)
    tr_b, buf_b, parts_b = b.planner.take_step_moves()
    assert np.array_equal(tr_a, tr_b) and parts_a == parts_b and np.array_equal(buf_a, buf_b)
    assert b.planner.free_queue() == a.planner.free_queue()
    quotas = (256, 64, 64, 128, 128, 128)
    for seed in range(3):
        steps, _ = make_schedule(seed, 4, 512, 256, quotas, max_prompt=3 * 512, max_closed=3)
        perm = np.random.default_rng(100 + seed).permutation(np.arange(1, 4000)).astype(np.int32)
        pa = KVPlanner(4000, len(quotas), PAGE, free_order=perm, op_rows=op_rows)
        pb = KVPlanner(4000, len(quotas), PAGE, free_order=perm, op_rows=op_rows)
        seen_a, seen_b = set(), set()
        from tests.planner_harness import run_events
        for events in steps:
            out = run_native_step(pa, events, seen_a)
            run_events(pb, events, seen_b)
            tr, buf, parts = pb.take_step_moves()
            fm = np.asarray(out.fused_moves, dtype=np.int64)
            ref_buf, ref_parts = worker.pack_fused_moves(fm, 4000, num_groups=len(quotas)) if fm.size else (None, [])
            assert parts == ref_parts
            if parts:
                assert np.array_equal(buf, ref_buf)
            assert {pb.request_id(int(r[0])): tuple(int(x) for x in r[1:]) for r in tr} == out.block_table_truncations


def test_config2_fused_moves_equal_oracle_batches():
    """The 64-sequence compaction step: the native planner's fused moves (gather-then-scatter per group) and the
    oracle planner's ordered op batches (oracle.compaction.execute_kv_copy_operations, the reference executor's
    batch order, gpu_model_runner.py:1147-1224), both applied to a row-id image of the pool (every slot holds its own
    id), leave every kept row of every request and group holding the same id; the page lists and compacted counts
    of both planners agree."""
    from oracle import compaction as oc

    st = workloads.build_compaction_state(64, seed=0, op_rows=False)
    G = len(st.groups)
    orc = oc.Planner(st.num_pages, G, PAGE, free_order=st.free_order)
    orc.apply_events(st.history)
    orc.take_step_outputs()
    orc.apply_events(st.pending)
    batches, _ = orc.take_step_outputs()
    out = st.compact()
    fused = np.asarray(out.fused_moves, np.int64)
    assert fused.size and len(batches) == 64
    image = np.arange(st.num_pages * PAGE, dtype=np.int64).reshape(st.num_pages, PAGE)
    kept_rows = 0
    for g in range(G):
        mine = gather_then_scatter(image, fused[fused[:, 1] == g])
        ref = np.stack([image, image], axis=1).copy()                 # [pages, 2 (K, V), 16]
        oc.execute_kv_copy_operations({r: b for r, b in batches.items()},
                                      [[ref] if i == g else [] for i in range(G)])
        assert np.array_equal(ref[:, 0], ref[:, 1])
        for r in range(64):
            blocks = st.planner.get_blocks(r)[g]
            assert blocks == orc.block_ids(r)[g]
            assert st.planner.compacted_counts(r)[g] == orc.requests[r].compacted_counts()[g]
            active = st.planner.num_computed_tokens(r) - st.planner.compacted_counts(r)[g]
            slots = oc.slot_mapping(blocks, np.arange(active))
            got, want = mine[slots // PAGE, slots % PAGE], ref[slots // PAGE, 0, slots % PAGE]
            assert np.array_equal(got, want), (r, g)
            kept_rows += active
    assert kept_rows > 64 * G * 128
