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
