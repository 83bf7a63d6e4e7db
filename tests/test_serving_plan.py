"""The serving loop's host half (ServingPlan) without a GPU: the state machine settles every step through the planner,
and each step's compaction moves come out of the planner as run descriptors, expanded here with the host restatement
of the device expansion into the mixed launch's move lists. Every list, run through the CPU model of the mixed launch
(random interleavings of the workgroups' load and store phases), equals gather-then-scatter of its own ops -- the
ordering the lists promise holds on the moves the loop really produces."""
import numpy as np

from tests.test_move_pack import gather_then_scatter, phases, run_model, unpack
from tests.test_move_runs import expand


def test_serving_plan_moves_are_exact_under_any_interleaving():
    from abridgekv_amd.serving import ServingPlan
    rng = np.random.default_rng(0)
    B, C, K = 8, 64, 16
    quotas = (16, 4, 8, 4, 16, 8)
    T = rng.integers(200, 600, B)
    P = rng.integers(10, 150, B)
    plan = ServingPlan(T, P, layer_quotas=quotas, seed=0, growth_tokens=256, C=C, K=K)
    cache = rng.integers(0, 1 << 30, size=(plan.st.num_pages, 16))
    n_lists = n_ordered = 0
    for _ in range(150):
        moves = plan.advance(plan.prepare())
        if moves is None:
            continue
        kind, desc, layout, parts, n_elems = moves
        assert kind == "runs"                               # the loop's steps stay within the descriptors' limits
        buf = expand(desc, layout, n_elems, plan.G)
        for gid, (ops_g, offs, nf) in unpack(buf, parts).items():
            rows = np.concatenate([np.zeros((len(ops_g), 2), np.int64), ops_g.astype(np.int64)], axis=1)
            ref = gather_then_scatter(cache, rows)
            assert np.array_equal(run_model(cache, ops_g, phases(ops_g, offs, nf), rng), ref)
            n_lists += 1
            n_ordered += len(offs) - 1
    assert n_lists > 0 and plan.stats["moved_rows"] > 0
    assert plan.stats["code_steps"] >= B
