"""Drive the oracle planner and the native planner with the same scheduler event stream and compare them."""
from __future__ import annotations

import numpy as np

from oracle import compaction as oc
from oracle import trace as ot


def run_oracle_step(planner: oc.Planner, events, added: set):
    for ev in events:
        if ev[0] == "alloc":
            _, rid, n = ev
            if rid not in added:
                planner.add_request(rid)
                added.add(rid)
            assert planner.allocate_slots(rid, n) is not None, "oracle pool exhausted"
            planner.requests[rid].num_computed_tokens += n
        else:
            _, rid, s, e, g = ev
            res = planner.mask_token_span(rid, s, e, g)
            assert res.success, res.error_message
    return planner.take_step_outputs()


def run_native_step(planner, events, added: set):
    run_events(planner, events, added)
    return planner.take_step_outputs()


def run_events(planner, events, added: set) -> None:
    """A step's allocations and span removals on the native planner (outputs left pending)."""
    for ev in events:
        if ev[0] == "alloc":
            _, rid, n = ev
            if rid not in added:
                planner.add_request(rid)
                added.add(rid)
            assert planner.allocate_slots(rid, n) is not None, "native pool exhausted"
            planner.set_num_computed_tokens(rid, planner.num_computed_tokens(rid) + n)
        else:
            _, rid, s, e, g = ev
            res = planner.mask_token_span(rid, s, e, g)
            assert res.success, res.error_message


def events_to_array(steps, num_groups):
    """Flatten a build_schedule event list into abkv_planner_apply_events rows."""
    rows, added = [], set()
    for events in steps:
        for ev in events:
            if ev[0] == "alloc":
                if ev[1] not in added:
                    rows.append((0, ev[1], 0, 0, 0, 0))
                    added.add(ev[1])
                rows.append((1, ev[1], ev[2], 0, 0, 0))
            else:
                g = ev[4]
                mask = -1 if g is None else sum(1 << x for x in g)
                rows.append((2, ev[1], ev[2], ev[3], mask, 0))
        rows.append((4, 0, 0, 0, 0, 0))
    return np.asarray(rows, dtype=np.int64)


def compare_state(oracle: oc.Planner, native, rids):
    assert oracle.pool.free_queue.order() == native.free_queue(), "free queue order differs"
    for rid in rids:
        assert tuple(oracle.block_ids(rid)) == native.get_blocks(rid), f"page lists differ for {rid}"
        assert oracle.requests[rid].compacted_counts() == native.compacted_counts(rid)
        for g in range(oracle.num_groups):
            assert oracle.requests[rid].groups[g].spans == native.group_compacted_spans(rid, g)


def make_schedule(seed, n_req, C, K, quotas, max_prompt, max_closed, num_steps=None):
    """Requests with seeded prompts that start staggered so their block closings interleave."""
    rng = np.random.default_rng(seed)
    prompts = rng.integers(1, max_prompt + 1, n_req).tolist()
    starts = rng.integers(0, 8, n_req).tolist()
    closes = [ot.steps_until_closed(p, max_closed, C, K, quotas) for p in prompts]
    total = num_steps if num_steps is not None else max(s + c for s, c in zip(starts, closes)) + 3
    return ot.build_schedule(prompts, [1 << 30] * n_req, starts, total, C, K, quotas)



def apply_events_oracle(planner: oc.Planner, rows) -> None:
    """abkv_planner_apply_events rows through the oracle planner."""
    planner.apply_events(rows)
