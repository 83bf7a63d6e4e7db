"""Compaction on the GPU: the native planner + HIP row mover reproduce, bit for bit, the reference's semantics
executed by the oracle on CPU copies of the same caches (gather-then-scatter per batch, group by group), and every
kept row holds the bytes written for its logical token."""
import numpy as np
import pytest
import torch

from abridgekv_amd import ops, worker
from abridgekv_amd.planner import KVPlanner
from oracle import compaction as oc
from tests.planner_harness import make_schedule

pytestmark = pytest.mark.gpu

# Six groups with the served 4:1:1:2:2:2 quota pattern on a shorter block (C=128, K=64) so the schedule stays short;
# the planner itself is checked on the served C=512 / K=256 geometry in tests/test_planner_native.py.
C_BLOCK, K_CODES = 128, 64
QUOTAS = (64, 16, 16, 32, 32, 32)
LAYERS_PER_GROUP = 2


def row_content(rid, positions, layer):
    """Identifiable [n, 2, 8, 128] bf16 rows (as int16 bit patterns): each 16-byte vector holds
    (rid, position, layer, vector index) -- any misplaced or stale row is detected."""
    positions = np.asarray(positions, dtype=np.int32)
    n = positions.size
    vec = np.arange(256, dtype=np.int32)                      # 2 x 2048 B / 16 B vectors per row
    q = np.empty((n, 256, 4), np.int32)
    q[..., 0] = rid
    q[..., 1] = positions[:, None]
    q[..., 2] = layer
    q[..., 3] = vec[None, :]
    return q.view(np.int16).reshape(n, 2, 8, 128)


def _write_tokens(cache_np, gpu_caches, slots, rows):
    """KV append of a step's new rows: numpy reference write + the HIP append kernel on each GPU cache."""
    pages, offs = slots // 16, slots % 16
    cache_np[pages, :, offs] = rows
    rows_t = torch.from_numpy(np.ascontiguousarray(rows)).view(torch.bfloat16).to(gpu_caches[0].device)
    k, v = rows_t[:, 0].contiguous(), rows_t[:, 1].contiguous()
    slots_d = torch.from_numpy(slots.astype(np.int64)).to(gpu_caches[0].device)
    for c in gpu_caches:
        ops.kv_append(k, v, slots_d, c)


@pytest.mark.parametrize("seed", [0, 1])
def test_compaction_matches_oracle_bit_exact(seed):
    steps, traces = make_schedule(seed, 5, C_BLOCK, K_CODES, QUOTAS, max_prompt=300, max_closed=3)
    G = len(QUOTAS)
    num_pages = 2048
    perm = np.random.default_rng(seed).permutation(np.arange(1, num_pages)).astype(np.int32)
    native = KVPlanner(num_pages, G, 16, free_order=perm)
    oracle = oc.Planner(num_pages, G, 16, free_order=perm)
    dev = torch.device("cuda")
    # tensor i holds layer i of every group (kv_cache_utils.py:1110-1127)
    np_caches = [np.zeros((num_pages, 2, 16, 8, 128), np.int16) for _ in range(LAYERS_PER_GROUP)]
    ref_gpu = [torch.zeros(ops.kv_cache_shape(num_pages), dtype=torch.bfloat16, device=dev)
               for _ in range(LAYERS_PER_GROUP)]
    fused_gpu = [torch.zeros_like(c) for c in ref_gpu]
    by_group_ref = [ref_gpu] * G
    by_group_fused = [fused_gpu] * G
    pending_o = pending_n = None
    added = set()
    n_moves = 0
    for events in steps + [[]]:
        if pending_n is not None:
            oc.execute_kv_copy_operations(pending_o, [np_caches] * G)
            worker.execute_kv_copy_operations(pending_n.kv_copy_operations, by_group_ref)
            worker.execute_fused_moves(pending_n.fused_moves, by_group_fused)
            n_moves += len(pending_n.fused_moves)
        writes = [([], []) for _ in range(LAYERS_PER_GROUP)]
        for ev in events:
            if ev[0] != "alloc":
                continue
            _, rid, n = ev
            if rid not in added:
                native.add_request(rid)
                oracle.add_request(rid)
                added.add(rid)
            assert native.allocate_slots(rid, n) is not None
            assert oracle.allocate_slots(rid, n) is not None
            start = native.num_computed_tokens(rid)
            logical = np.arange(start, start + n)
            phys = worker.physical_positions(logical, native.compacted_counts(rid))
            blocks = native.get_blocks(rid)
            for g in range(G):
                slots = worker.slot_mapping_host(blocks[g], phys[g])
                assert np.array_equal(slots, oc.slot_mapping(oracle.block_ids(rid)[g], phys[g]))
                for i in range(LAYERS_PER_GROUP):
                    writes[i][0].append(slots)
                    writes[i][1].append(row_content(rid, logical, g * 16 + i))
            native.set_num_computed_tokens(rid, start + n)
            oracle.requests[rid].num_computed_tokens += n
        for i in range(LAYERS_PER_GROUP):
            if writes[i][0]:
                _write_tokens(np_caches[i], [ref_gpu[i], fused_gpu[i]], np.concatenate(writes[i][0]),
                              np.concatenate(writes[i][1]))
        for ev in events:
            if ev[0] == "mask":
                _, rid, s, e, g = ev
                assert native.mask_token_span(rid, s, e, g).success
                assert oracle.mask_token_span(rid, s, e, g).success
        pending_n = native.take_step_outputs()
        pending_o, _ = oracle.take_step_outputs()
    torch.cuda.synchronize()
    assert n_moves > 0
    # 1) reference-format ops on the GPU == oracle execution on the CPU, every byte of every page
    for i in range(LAYERS_PER_GROUP):
        got = ref_gpu[i].view(torch.int16).cpu().numpy()
        assert np.array_equal(got, np_caches[i]), f"cache {i} differs from the oracle execution"
    # 2) fused moves: every kept row equals the oracle's, and holds its own logical token's bytes
    for rid in sorted(added):
        blocks = native.get_blocks(rid)
        for g in range(G):
            active = native.num_computed_tokens(rid) - native.compacted_counts(rid)[g]
            phys = np.arange(active)
            slots = worker.slot_mapping_host(blocks[g], phys)
            logical = np.array([native.physical_to_logical(rid, x, g) for x in phys])
            kept = traces[rid].kept_positions(g)
            assert len(kept) == active and logical.tolist() == kept
            for i in range(LAYERS_PER_GROUP):
                got = fused_gpu[i].view(torch.int16)[torch.from_numpy(slots // 16).to(dev), :,
                                                     torch.from_numpy(slots % 16).to(dev)].cpu().numpy()
                assert np.array_equal(got, np_caches[i][slots // 16, :, slots % 16])
                assert np.array_equal(got, row_content(rid, logical, g * 16 + i))


def test_staged_copy_handles_overlapping_chains():
    """An op list where later ops read slots earlier ops wrote must still act as gather-then-scatter."""
    dev = torch.device("cuda")
    cache = torch.zeros(ops.kv_cache_shape(8), dtype=torch.bfloat16, device=dev)
    rows = row_content(9, np.arange(8 * 16), 0)
    cache.view(torch.int16).copy_(torch.from_numpy(rows.reshape(8, 16, 2, 8, 128).transpose(0, 2, 1, 3, 4).copy()))
    before = cache.view(torch.int16).cpu().numpy().copy()
    ops_l = [(1, 0, 2, 0), (2, 0, 3, 0), (3, 0, 1, 0), (5, 5, 5, 4), (5, 4, 5, 3)]   # a cycle and a right shift
    worker.execute_kv_copy_group([ops_l], [cache])
    torch.cuda.synchronize()
    expect = before.copy()
    src = np.array(ops_l)
    expect[src[:, 2], :, src[:, 3]] = before[src[:, 0], :, src[:, 1]]
    assert np.array_equal(cache.view(torch.int16).cpu().numpy(), expect)


def test_full_size_compaction_moves_every_row_exactly():
    """The served geometry at full size (64 sequences close a 512-token block with 256 code rows, 6 quota groups): the
    fused moves of one planner step, applied by the mover to a cache whose every 4-byte word carries its own address,
    leave each destination row equal, word for word, to the row that gather-then-scatter per (request, group)
    assigns it, and leave a sample of untouched rows unchanged."""
    from abridgekv_amd import workloads
    st = workloads.build_compaction_state(64, seed=0)
    _, _, fused = st.compact(as_arrays=True)
    fused = np.asarray(fused, np.int64)
    P = st.num_pages
    dev = torch.device("cuda")
    words = 2 * 16 * 512                                          # int32 words per page ([2][16 slots][512])
    assert P * words < 2 ** 31
    tag = torch.arange(P * words, dtype=torch.int32, device=dev)
    cache = tag.view(torch.bfloat16).view(ops.kv_cache_shape(P))   # every word holds its own linear index
    worker.execute_fused_moves(fused, [[cache] for _ in st.groups])
    torch.cuda.synchronize()
    # expected origin of every written row: gather-then-scatter per (request, group) segment, in order
    origin = {}
    for (r, g), rows in _segments(fused):
        srcs = [origin.get((int(a), int(b)), (int(a), int(b))) for a, b in rows[:, 2:4]]
        for (dp, ds), src in zip(rows[:, 4:6], srcs):
            origin[(int(dp), int(ds))] = src
    dst = np.array(list(origin.keys()), np.int64)
    src = np.array([origin[k] for k in origin], np.int64)
    got = tag.view(P, 2, 16, 512)[torch.from_numpy(dst[:, 0]).to(dev), :, torch.from_numpy(dst[:, 1]).to(dev)]
    half = np.arange(2)[None, :, None]
    word = np.arange(512)[None, None, :]
    want = ((src[:, 0, None, None] * 2 + half) * 16 + src[:, 1, None, None]) * 512 + word
    assert np.array_equal(got.cpu().numpy(), want)
    rng = np.random.default_rng(1)
    written = set(origin)
    sample = [(int(p), int(s)) for p, s in zip(rng.integers(0, P, 4000), rng.integers(0, 16, 4000))
              if (int(p), int(s)) not in written]
    sp = np.array(sample, np.int64)
    got = tag.view(P, 2, 16, 512)[torch.from_numpy(sp[:, 0]).to(dev), :, torch.from_numpy(sp[:, 1]).to(dev)]
    want = ((sp[:, 0, None, None] * 2 + half) * 16 + sp[:, 1, None, None]) * 512 + word
    assert np.array_equal(got.cpu().numpy(), want)


def _segments(fused):
    """(request, group) runs of a planner step's fused move rows, in order."""
    cut = np.flatnonzero(np.any(np.diff(fused[:, :2], axis=0) != 0, axis=1)) + 1
    for rows in np.split(fused, cut):
        yield (int(rows[0, 0]), int(rows[0, 1])), rows
