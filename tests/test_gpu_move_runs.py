"""The device half of the planner's fused moves (abkv_moves_expand over abkv_planner_take_move_runs' descriptors)
writes exactly the move lists the planner writes row by row on the host (abkv_planner_take_moves_packed), and the
mover fed from either leaves the same cache: on the 64-sequence compaction step and on multi-step served schedules."""
import numpy as np
import pytest
import torch

from abridgekv_amd import ops, worker, workloads
from abridgekv_amd.planner import KVPlanner
from tests.planner_harness import make_schedule, run_events

pytestmark = pytest.mark.gpu

PAGE = 16


def _host_and_device(pa, pb, dev, up_runs):
    """(host-written buffer, device-expanded buffer as numpy, parts) for the pending steps of two equal planners."""
    tr_a, buf_a, parts_a = pa.take_step_moves()
    tr_b, lists = up_runs.take(pb)
    assert np.array_equal(tr_a, tr_b)
    torch.cuda.synchronize()
    return buf_a, up_runs._out[:buf_a.size].cpu().numpy(), parts_a, lists


def test_expansion_equals_host_lists_on_the_64_sequence_step():
    dev = torch.device("cuda")
    a = workloads.build_compaction_state(64, seed=0, op_rows=False)
    b = workloads.build_compaction_state(64, seed=0, op_rows=False)
    a.planner.apply_events(a.pending)
    b.planner.apply_events(b.pending)
    up = worker.MoveRunUploader(dev, capacity=1 << 10, out_capacity=1 << 10)   # both buffers grow on first use
    print("case: 64-sequence step", flush=True)
    buf_a, got, parts, _ = _host_and_device(a.planner, b.planner, dev, up)
    assert parts and np.array_equal(got, buf_a)
    assert a.planner.free_queue() == b.planner.free_queue()


@pytest.mark.parametrize("seed", range(3))
def test_expansion_equals_host_lists_on_served_schedules(seed):
    dev = torch.device("cuda")
    quotas = (256, 64, 64, 128, 128, 128)
    steps, _ = make_schedule(seed, 4, 512, 256, quotas, max_prompt=3 * 512, max_closed=3)
    perm = np.random.default_rng(100 + seed).permutation(np.arange(1, 4000)).astype(np.int32)
    pa = KVPlanner(4000, len(quotas), PAGE, free_order=perm, op_rows=False)
    pb = KVPlanner(4000, len(quotas), PAGE, free_order=perm, op_rows=False)
    up = worker.MoveRunUploader(dev)
    seen_a, seen_b = set(), set()
    checked = 0
    print(f"case: schedule seed {seed}", flush=True)
    for events in steps:
        run_events(pa, events, seen_a)
        run_events(pb, events, seen_b)
        buf_a, got, parts, _ = _host_and_device(pa, pb, dev, up)
        if parts:
            assert np.array_equal(got, buf_a)
            checked += 1
    assert checked >= 3


def test_mover_fed_from_device_lists_leaves_the_same_cache():
    """Full size: the 64-sequence step's moves applied once from the host-written lists and once from the device
    expansion, each to its own copy of a cache whose every 4-byte word carries its own address."""
    dev = torch.device("cuda")
    a = workloads.build_compaction_state(64, seed=0, op_rows=False)
    b = workloads.build_compaction_state(64, seed=0, op_rows=False)
    a.planner.apply_events(a.pending)
    b.planner.apply_events(b.pending)
    P = a.num_pages
    words = 2 * 16 * 512
    assert P * words < 2 ** 31
    tag_a = torch.arange(P * words, dtype=torch.int32, device=dev)
    tag_b = tag_a.clone()
    cache_a = tag_a.view(torch.bfloat16).view(ops.kv_cache_shape(P))
    cache_b = tag_b.view(torch.bfloat16).view(ops.kv_cache_shape(P))
    print("case: full-size mover from both lists", flush=True)
    _, prepared_a = worker.MoveUploader(dev, capacity=8 << 20).take(a.planner)
    _, prepared_b = worker.MoveRunUploader(dev).take(b.planner)
    worker.launch_moves(prepared_a, [[cache_a] for _ in a.groups])
    worker.launch_moves(prepared_b, [[cache_b] for _ in b.groups])
    torch.cuda.synchronize()
    assert torch.equal(tag_a, tag_b)
    assert not torch.equal(tag_a, torch.arange(P * words, dtype=torch.int32, device=dev))   # rows did move


def test_expansion_of_eight_scrambled_removals():
    """Eight span removals of one request in one step, in a scrambled order (the row map's largest case)."""
    dev = torch.device("cuda")
    pa, pb = (KVPlanner(200, 1, PAGE, op_rows=False) for _ in range(2))
    for p in (pa, pb):
        p.add_request(7)
        assert p.allocate_slots(7, 1000) is not None
        p.set_num_computed_tokens(7, 1000)
        for k in range(8):
            s = 40 + 100 * ((5 * k) % 8)
            assert p.mask_token_span(7, s, s + 10 + k).success
    print("case: eight removals", flush=True)
    buf_a, got, parts, _ = _host_and_device(pa, pb, dev, worker.MoveRunUploader(dev))
    assert parts and np.array_equal(got, buf_a)
