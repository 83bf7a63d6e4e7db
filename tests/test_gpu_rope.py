"""Fused rotary embedding + KV append on the GPU.

The kernel computes in fp32 from bf16 inputs and the fp32 cos/sin table and rounds once to bf16, so each output is
pinned to the float64 rotation of the same inputs within half a bf16 ulp (2^-8 relative, plus fp32 slack); cache
rows are bit-identical to the rotated key and to value."""
import numpy as np
import pytest
import torch

from oracle import layout as ol

pytestmark = pytest.mark.gpu


def _rotate_fp64(x, pos, table):
    """NeoX rotation of x [T, H, 128] at RoPE positions pos [T] with table [P, 128] (cos | sin), in float64."""
    x = x.double()
    c = table[pos][:, None, :64].double()
    s = table[pos][:, None, 64:].double()
    x1, x2 = x[..., :64], x[..., 64:]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)


def _within_half_ulp(got, want):
    got = got.double()
    return bool(((got - want).abs() <= want.abs() * 2.0 ** -8 + 1e-6).all())


@pytest.mark.parametrize("logical,C,K,span", [(False, 64, 16, 0), (True, 64, 16, 0), (True, 48, 16, 0),
                                              (True, 64, 16, 52)])
def test_rotation_and_cache_rows(logical, C, K, span):
    """Plain RoPE positions, and logical positions of the abridged layout mapped on the device (also with a block
    size that is not a power of two: only the code count must be one; and with the code rows spread over the first
    span offsets, a static retained tail of C - span rows)."""
    from abridgekv_amd import ops
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(11)
    T, max_pos = 300, 8192
    q = torch.randn((T, 32, 128), generator=g).to(torch.bfloat16)
    k = (torch.randn((T, 8, 128), generator=g) * 3).to(torch.bfloat16)
    v = torch.randn((T, 8, 128), generator=g).to(torch.bfloat16)
    if logical:
        lpos = torch.randint(0, 90 * (C + K), (T,), generator=g)
        rpos = torch.from_numpy(ol.bitrev_rope_positions(lpos.numpy(), C, K, span or None))
    else:
        lpos = rpos = torch.randint(0, max_pos, (T,), generator=g)
    table = ops.rope_cos_sin_cache(max_pos)
    num_pages = 64
    perm = torch.randperm(num_pages * 16, generator=g)[:T]
    slots = perm.clone()
    slots[::7] = -1                                      # skipped rows
    cache = torch.randn((num_pages, 2, 16, 8, 128), generator=g).to(torch.bfloat16)
    qd, kd, vd, cd = q.to(dev), k.to(dev), v.to(dev), cache.to(dev)
    ops.rope_kv_append(qd, kd, vd, lpos.to(dev), table.to(dev), slot_mapping=slots.to(dev), kv_cache=cd,
                       block_c=C if logical else 0, codes_k=K if logical else 0, code_span=span)
    torch.cuda.synchronize()
    assert _within_half_ulp(qd.cpu(), _rotate_fp64(q, rpos, table))
    assert _within_half_ulp(kd.cpu(), _rotate_fp64(k, rpos, table))
    cc = cd.cpu()
    ok = slots >= 0
    pg, off = slots[ok] // 16, slots[ok] % 16
    assert torch.equal(cc[pg, 0, off], kd.cpu()[ok])
    assert torch.equal(cc[pg, 1, off], v[ok])
    untouched = torch.ones(num_pages * 16, dtype=torch.bool)
    untouched[slots[ok]] = False
    flat_new = cc.permute(0, 2, 1, 3, 4).reshape(num_pages * 16, 2, 8, 128)
    flat_old = cache.permute(0, 2, 1, 3, 4).reshape(num_pages * 16, 2, 8, 128)
    assert torch.equal(flat_new[untouched], flat_old[untouched])


def test_positions_past_the_table_are_rejected_on_the_host():
    """A cos/sin table shorter than the largest RoPE position raises before any launch (no silent clamping)."""
    from abridgekv_amd import ops
    dev = torch.device("cuda")
    q = torch.zeros((2, 32, 128), dtype=torch.bfloat16, device=dev)
    k = torch.zeros((2, 8, 128), dtype=torch.bfloat16, device=dev)
    table = ops.rope_cos_sin_cache(100).to(dev)
    with pytest.raises(ValueError, match="cos/sin table"):
        ops.rope_kv_append(q, k, k.clone(), torch.tensor([3, 100], device=dev), table)
    with pytest.raises(ValueError, match="cos/sin table"):        # logical 260 = block 3, content row 20 -> 212
        ops.rope_kv_append(q, k, k.clone(), torch.tensor([0, 260], device=dev), ops.rope_cos_sin_cache(212).to(dev),
                           block_c=64, codes_k=16, max_position=260)
    ops.rope_kv_append(q, k, k.clone(), torch.tensor([0, 260], device=dev), ops.rope_cos_sin_cache(213).to(dev),
                       block_c=64, codes_k=16, max_position=260)
    torch.cuda.synchronize()
