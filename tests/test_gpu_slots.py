"""Device slot mapping of a KV-cache group vs the host restatement (bit-exact): physical positions = logical -
compacted[request], slots from the group's block table, -1 outside the table."""
import numpy as np
import pytest
import torch

from abridgekv_amd import worker

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("with_compacted", [False, True])
def test_slot_mapping_matches_host(with_compacted):
    from abridgekv_amd import ops
    rng = np.random.default_rng(5)
    B, W, n = 9, 40, 3000
    table = rng.integers(1, 5000, (B, W)).astype(np.int32)
    comp = rng.integers(0, 300, B).astype(np.int32) if with_compacted else np.zeros(B, np.int32)
    req = rng.integers(-1, B + 1, n).astype(np.int32)                 # includes invalid request indices
    pos = rng.integers(-20, W * 16 + 320, n).astype(np.int64)           # includes positions off both ends
    want = np.full(n, -1, np.int64)
    for t in range(n):
        r = req[t]
        if 0 <= r < B:
            p = worker.physical_positions([pos[t]], [comp[r]])[0][0]
            if 0 <= p < W * 16:
                want[t] = worker.slot_mapping_host(table[r], [p])[0]
    dev = torch.device("cuda")
    got = ops.slot_mapping(torch.from_numpy(req).to(dev), torch.from_numpy(pos).to(dev),
                           torch.from_numpy(table).to(dev),
                           compacted=torch.from_numpy(comp).to(dev) if with_compacted else None)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("seed", [0, 3])
def test_slot_mapping_matches_oracle_planner(seed):
    """Device slot map of every step's new tokens, read through the native planner's block tables and compacted
    counts, equals oracle.compaction.slot_mapping over the oracle planner's page lists at the oracle's physical
    positions (logical - compacted per group, gpu_model_runner.py:1585-1590), across a schedule whose blocks close
    and compact; the native planner's physical positions equal the oracle's."""
    from abridgekv_amd import ops
    from abridgekv_amd.planner import KVPlanner
    from oracle import compaction as oc
    from tests.planner_harness import make_schedule

    C, K, quotas = 128, 64, (64, 16, 16, 32, 32, 32)
    G = len(quotas)
    steps, _ = make_schedule(seed, 6, C, K, quotas, max_prompt=300, max_closed=3)
    num_pages = 2048
    perm = np.random.default_rng(seed).permutation(np.arange(1, num_pages)).astype(np.int32)
    native = KVPlanner(num_pages, G, 16, free_order=perm)
    orc = oc.Planner(num_pages, G, 16, free_order=perm)
    dev = torch.device("cuda")
    added, rids = set(), []
    checked = 0
    W = 128
    for events in steps:
        toks = []
        for ev in events:
            if ev[0] != "alloc":
                continue
            _, rid, n = ev
            if rid not in added:
                native.add_request(rid)
                orc.add_request(rid)
                added.add(rid)
                rids.append(rid)
            assert native.allocate_slots(rid, n) is not None and orc.allocate_slots(rid, n) is not None
            start = orc.requests[rid].num_computed_tokens
            toks.append((rid, np.arange(start, start + n)))
            native.set_num_computed_tokens(rid, start + n)
            orc.requests[rid].num_computed_tokens += n
        if toks:
            idx = {r: i for i, r in enumerate(rids)}
            req = np.concatenate([np.full(len(lp), idx[r], np.int32) for r, lp in toks])
            pos = np.concatenate([lp for _, lp in toks]).astype(np.int64)
            for g in range(G):
                want = np.concatenate([oc.slot_mapping(orc.block_ids(r)[g], orc.physical_positions(r, lp)[g])
                                       for r, lp in toks])
                for r, lp in toks:
                    assert np.array_equal(worker.physical_positions(lp, native.compacted_counts(r))[g],
                                          orc.physical_positions(r, lp)[g])
                table = native.fill_block_table(rids, g, W)
                comp = np.array([native.compacted_counts(r)[g] for r in rids], np.int32)
                got = ops.slot_mapping(torch.from_numpy(req).to(dev), torch.from_numpy(pos).to(dev),
                                       torch.from_numpy(table).to(dev), compacted=torch.from_numpy(comp).to(dev))
                torch.cuda.synchronize()
                assert np.array_equal(got.cpu().numpy(), want), (g, events)
                checked += want.size
        for ev in events:
            if ev[0] == "mask":
                _, rid, s, e, gs = ev
                assert native.mask_token_span(rid, s, e, gs).success and orc.mask_token_span(rid, s, e, gs).success
        native.take_step_outputs()
        orc.take_step_outputs()
    assert checked > 1000 and any(native.compacted_counts(r)[0] for r in rids)
