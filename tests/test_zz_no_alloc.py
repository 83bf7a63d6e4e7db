"""The allocation-free decode entry point (abkv_decode_attn_noalloc, static device scratch) against abkv_decode_attn
with a caller workspace: both run the same kernels, so outputs and LSE must be bit-identical. Two calls in a row, the
second with a smaller batch and shorter sequences (the scratch keeps the first call's partials, which must not leak
into the second), plus a batch whose partials exceed the scratch (rejected, nothing launched)."""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _state(B, max_rows, seed, dev):
    rng = np.random.default_rng(seed)
    lens = rng.integers(1, max_rows + 1, B).astype(np.int32)
    lens[0] = max_rows
    W = -(-max_rows // 16)
    pages = rng.permutation(np.arange(1, B * W + 1)).astype(np.int32).reshape(B, W)
    return torch.from_numpy(lens).to(dev), torch.from_numpy(pages).to(dev), W


def _noalloc(q, cache, bt, sl, max_pages, split, out, lse):
    from abridgekv_amd import ops
    from abridgekv_amd._lib import lib
    return lib().abkv_decode_attn_noalloc(
        C.c_void_p(q.data_ptr()), q.stride(0), q.stride(1), C.c_void_p(cache.data_ptr()), cache.shape[0],
        C.c_void_p(bt.data_ptr()), bt.stride(0), C.c_void_p(sl.data_ptr()), q.shape[0], max_pages, split,
        C.c_float(ops.default_scale()), C.c_void_p(out.data_ptr()), out.stride(0), out.stride(1),
        C.c_void_p(lse.data_ptr()), C.c_void_p(torch.cuda.current_stream().cuda_stream))


def test_noalloc_matches_workspace_entry_point_twice():
    from abridgekv_amd import ops
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(21)
    cache = torch.empty(ops.kv_cache_shape(256 * 140 + 1), dtype=torch.bfloat16, device=dev)
    cache.normal_(generator=gen)
    for B, max_rows, split, seed in ((256, 2200, 8, 1), (37, 700, 4, 2)):
        sl, bt, W = _state(B, max_rows, seed, dev)
        q = torch.randn((B, 32, 128), generator=gen, device=dev).to(torch.bfloat16)
        ref_o = torch.empty((B, 32, 128), dtype=torch.bfloat16, device=dev)
        ref_l = torch.empty((B, 32), dtype=torch.float32, device=dev)
        ops.decode_attention(q, cache, bt, sl, ops.default_scale(), max_pages=W, out=ref_o, lse=ref_l,
                             split_pages=split)
        out = torch.full((B, 32, 128), 3.0, dtype=torch.bfloat16, device=dev)
        lse = torch.full((B, 32), 3.0, dtype=torch.float32, device=dev)
        assert _noalloc(q, cache, bt, sl, W, split, out, lse) == 0
        torch.cuda.synchronize()
        assert -(-W // split) > 1                                        # the partials path is exercised
        assert torch.equal(out, ref_o), (B, max_rows)
        assert torch.equal(lse, ref_l), (B, max_rows)


def test_noalloc_rejects_batches_beyond_the_scratch():
    from abridgekv_amd import ops
    from abridgekv_amd._lib import lib
    dev = torch.device("cuda")
    B, W, split = 256, 2048, 2                                          # 1024 splits x 256 seqs of partials
    assert lib().abkv_decode_workspace_size(B, W // split) > ops.DECODE_NOALLOC_SCRATCH_BYTES
    cache = torch.zeros(ops.kv_cache_shape(4), dtype=torch.bfloat16, device=dev)
    bt = torch.zeros((B, W), dtype=torch.int32, device=dev)
    sl = torch.ones(B, dtype=torch.int32, device=dev)
    q = torch.zeros((B, 32, 128), dtype=torch.bfloat16, device=dev)
    out = torch.full((B, 32, 128), 5.0, dtype=torch.bfloat16, device=dev)
    lse = torch.zeros((B, 32), dtype=torch.float32, device=dev)
    assert _noalloc(q, cache, bt, sl, W, split, out, lse) == ops.ABKV_ERR_SCRATCH
    with pytest.raises(ValueError, match="static scratch"):
        ops.decode_attention_noalloc(q, cache, bt, sl, ops.default_scale(), out, max_pages=W, split_pages=split)
    torch.cuda.synchronize()
    assert bool((out == 5.0).all())
