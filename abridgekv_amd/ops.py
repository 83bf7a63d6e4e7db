"""PyTorch-ROCm entry points of the abridged-KV kernels (thin wrappers over the C-ABI library).

Every wrapper validates shapes, dtypes and devices on the host before a launch, runs on the caller's current HIP
stream, never synchronises, and raises ``RuntimeError`` on a non-zero HIP error code. There is no CPU fallback:
tensors must live on a GPU and the native library must be built.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import torch

from ._lib import check, lib

PAGE = 16
HEADS_KV = 8
HEADS_Q = 32
HEAD_DIM = 128
SLOT_BYTES = HEADS_KV * HEAD_DIM * 2           # one slot of K (or V) of one layer, bf16
HALF_BYTES = PAGE * SLOT_BYTES                 # K half of a page
PAGE_BYTES = 2 * HALF_BYTES                    # one page of one layer
DEFAULT_SPLIT_PAGES = 32                       # 512 slots per split
AUTO_SPLIT_CHOICES = (48, 40, 32)               # pages per split the host may pick (a workspace for 32 fits all)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None):
    return None if t is None else C.c_void_p(t.data_ptr())


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def kv_cache_shape(num_pages: int) -> tuple[int, ...]:
    """Layer cache shape [num_pages, 2, 16, 8, 128] (the reference's FlashInfer NHD layout,
    third_party/vllm_overlay/vllm/v1/worker/gpu_model_runner.py:1215-1217)."""
    return (num_pages, 2, PAGE, HEADS_KV, HEAD_DIM)


def _row_stride(block_table: torch.Tensor) -> int:
    """Row stride of a [B, W] page table (a single row's stride is arbitrary in torch, e.g. 0 for a numpy
    ``table[None]`` view, so it is reported as W)."""
    W = block_table.shape[1]
    if block_table.shape[0] <= 1:
        return W
    _require(block_table.stride(0) >= W, "block_table rows must not overlap")
    return block_table.stride(0)


def _check_cache(kv_cache: torch.Tensor, dtype=torch.bfloat16) -> None:
    _require(kv_cache.is_cuda, "kv_cache must be on the GPU")
    _require(kv_cache.dtype == dtype, f"kv_cache must be {dtype}")
    _require(kv_cache.dim() == 5 and tuple(kv_cache.shape[1:]) == (2, PAGE, HEADS_KV, HEAD_DIM),
             f"kv_cache must be [P, 2, {PAGE}, {HEADS_KV}, {HEAD_DIM}], got {tuple(kv_cache.shape)}")
    _require(kv_cache.is_contiguous(), "kv_cache must be contiguous")


_NUM_CUS = None


def _num_cus() -> int:
    global _NUM_CUS
    if _NUM_CUS is None:
        _NUM_CUS = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count \
            if torch.cuda.is_available() else 256
    return _NUM_CUS


def auto_split_pages(seq_lens, num_cus: int | None = None) -> int:
    """Pages per decode split for a batch of host row counts: the largest of 48, 40, 32 whose grid still fills the GPU
    (four 2-wave workgroups per split, eight workgroups per CU). Longer splits write fewer partials; too few
    workgroups leave CUs idle. Measured: 48 on the B=256 saturated workload (1.1 % faster than 32), 40 on the B=64
    full-model decode (0.7 %), where 48 under-fills the GPU (1.7 % slower)."""
    pages = -(-np.asarray(seq_lens, dtype=np.int64) // PAGE)
    slots = 8 * (_num_cus() if num_cus is None else int(num_cus))
    for sp in AUTO_SPLIT_CHOICES:
        if 4 * int(np.maximum(1, -(-pages // sp)).sum()) >= slots:
            return sp
    return DEFAULT_SPLIT_PAGES


def decode_workspace(num_seqs: int, max_pages: int, split_pages: int = DEFAULT_SPLIT_PAGES,
                     device=None) -> torch.Tensor | None:
    """Workspace for :func:`decode_attention` (None when no sequence can need a second split)."""
    max_splits = -(-max_pages // split_pages)
    if max_splits <= 1:
        return None
    n = lib().abkv_decode_workspace_size(num_seqs, max_splits)
    return torch.empty(n, dtype=torch.uint8, device=device)


def decode_attention(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor,
                     scale: float, max_pages: int | None = None, out: torch.Tensor | None = None,
                     lse: torch.Tensor | None = None, split_pages: int = DEFAULT_SPLIT_PAGES,
                     workspace: torch.Tensor | None = None):
    """Decode attention of one layer over its group's paged cache.

    q [B, 32, 128] bf16 (dims contiguous); kv_cache [P, 2, 16, 8, 128] bf16; block_table [B, W] int32;
    seq_lens [B] int32 (physical rows); ``max_pages`` bounds ceil(seq_len / 16) (defaults to W).
    Writes and returns (out [B, 32, 128] bf16, lse [B, 32] fp32 natural log or None).
    fp32 q and cache select the fp32 mode (out fp32; split_pages and workspace unused).
    """
    if q.dtype == torch.float32:
        return _decode_attention_f32(q, kv_cache, block_table, seq_lens, scale, max_pages, out, lse)
    _check_cache(kv_cache)
    _require(q.is_cuda and q.dtype == torch.bfloat16 and q.dim() == 3 and tuple(q.shape[1:]) == (HEADS_Q, HEAD_DIM),
             f"q must be cuda bf16 [B, {HEADS_Q}, {HEAD_DIM}]")
    _require(q.stride(2) == 1, "q dims must be contiguous")
    B = q.shape[0]
    _require(block_table.is_cuda and block_table.dtype == torch.int32 and block_table.dim() == 2
             and block_table.shape[0] >= B and block_table.stride(1) == 1, "block_table must be cuda int32 [B, W]")
    _require(seq_lens.is_cuda and seq_lens.dtype == torch.int32 and seq_lens.numel() >= B
             and seq_lens.is_contiguous(), "seq_lens must be contiguous cuda int32 [B]")
    _require(0 < split_pages <= 64 and split_pages % 2 == 0, "split_pages must be an even number in [2, 64]")
    W = block_table.shape[1]
    max_pages = W if max_pages is None else int(max_pages)
    _require(0 < max_pages <= W, "max_pages must be in [1, block_table width]")
    if out is None:
        out = torch.empty((B, HEADS_Q, HEAD_DIM), dtype=torch.bfloat16, device=q.device)
    _require(out.dtype == torch.bfloat16 and tuple(out.shape) == (B, HEADS_Q, HEAD_DIM) and out.stride(2) == 1,
             "out must be bf16 [B, 32, 128] with contiguous dims")
    if lse is not None:
        _require(lse.dtype == torch.float32 and lse.is_contiguous() and lse.numel() >= B * HEADS_Q,
                 "lse must be contiguous fp32 [B, 32]")
    max_splits = -(-max_pages // split_pages)
    ws_bytes = 0
    if max_splits > 1:
        need = lib().abkv_decode_workspace_size(B, max_splits)
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
        _require(workspace.numel() * workspace.element_size() >= need, "decode workspace too small")
        ws_bytes = workspace.numel() * workspace.element_size()
    rc = lib().abkv_decode_attn(_ptr(q), q.stride(0), q.stride(1), _ptr(kv_cache), kv_cache.shape[0],
                                _ptr(block_table),
                                _row_stride(block_table), _ptr(seq_lens), B, max_pages, split_pages, float(scale),
                                _ptr(out), out.stride(0), out.stride(1), _ptr(lse), _ptr(workspace), ws_bytes,
                                C.c_void_p(_stream()))
    check(rc, "abkv_decode_attn")
    return out, lse


DECODE_NOALLOC_SCRATCH_BYTES = 64 << 20        # ABKV_DECODE_NOALLOC_SCRATCH_BYTES
ABKV_ERR_SCRATCH = -6


def decode_attention_noalloc(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor,
                             seq_lens: torch.Tensor, scale: float, out: torch.Tensor, max_pages: int | None = None,
                             lse: torch.Tensor | None = None, split_pages: int = DEFAULT_SPLIT_PAGES) -> None:
    """:func:`decode_attention` for callers that cannot allocate (graph capture, tight serving loops): nothing is
    allocated, the split partials use the library's static device scratch (64 MiB per GPU, shared by every call on
    that GPU, so calls overlapping on one GPU race). ``out`` (and ``lse`` if wanted) must be given. A batch whose
    partials exceed the scratch raises ValueError before any launch."""
    _check_cache(kv_cache)
    _require(q.is_cuda and q.dtype == torch.bfloat16 and q.dim() == 3 and tuple(q.shape[1:]) == (HEADS_Q, HEAD_DIM)
             and q.stride(2) == 1, f"q must be cuda bf16 [B, {HEADS_Q}, {HEAD_DIM}] with contiguous dims")
    B = q.shape[0]
    _require(block_table.is_cuda and block_table.dtype == torch.int32 and block_table.dim() == 2
             and block_table.shape[0] >= B and block_table.stride(1) == 1, "block_table must be cuda int32 [B, W]")
    _require(seq_lens.is_cuda and seq_lens.dtype == torch.int32 and seq_lens.numel() >= B
             and seq_lens.is_contiguous(), "seq_lens must be contiguous cuda int32 [B]")
    _require(0 < split_pages <= 64 and split_pages % 2 == 0, "split_pages must be an even number in [2, 64]")
    W = block_table.shape[1]
    max_pages = W if max_pages is None else int(max_pages)
    _require(0 < max_pages <= W, "max_pages must be in [1, block_table width]")
    _require(out is not None and out.dtype == torch.bfloat16 and tuple(out.shape) == (B, HEADS_Q, HEAD_DIM)
             and out.stride(2) == 1, "out must be given: bf16 [B, 32, 128] with contiguous dims")
    if lse is not None:
        _require(lse.dtype == torch.float32 and lse.is_contiguous() and lse.numel() >= B * HEADS_Q,
                 "lse must be contiguous fp32 [B, 32]")
    max_splits = -(-max_pages // split_pages)
    if max_splits > 1:
        need = lib().abkv_decode_workspace_size(B, max_splits)
        _require(need <= DECODE_NOALLOC_SCRATCH_BYTES,
                 f"{B} sequences x {max_splits} splits need {need} bytes of split partials, more than the "
                 f"{DECODE_NOALLOC_SCRATCH_BYTES}-byte static scratch (use longer splits or decode_attention)")
    rc = lib().abkv_decode_attn_noalloc(_ptr(q), q.stride(0), q.stride(1), _ptr(kv_cache), kv_cache.shape[0],
                                        _ptr(block_table), _row_stride(block_table), _ptr(seq_lens), B, max_pages,
                                        split_pages, float(scale), _ptr(out), out.stride(0), out.stride(1),
                                        _ptr(lse), C.c_void_p(_stream()))
    if rc == ABKV_ERR_SCRATCH:
        raise ValueError("abkv_decode_attn_noalloc: the batch needs more than the static scratch")
    check(rc, "abkv_decode_attn_noalloc")


def _decode_attention_f32(q, kv_cache, block_table, seq_lens, scale, max_pages, out, lse):
    _check_cache(kv_cache, torch.float32)
    _require(q.is_cuda and q.dim() == 3 and tuple(q.shape[1:]) == (HEADS_Q, HEAD_DIM) and q.stride(2) == 1,
             "q must be cuda fp32 [B, 32, 128] with contiguous dims")
    B = q.shape[0]
    _require(block_table.is_cuda and block_table.dtype == torch.int32 and block_table.dim() == 2
             and block_table.shape[0] >= B and block_table.stride(1) == 1, "block_table must be cuda int32 [B, W]")
    _require(seq_lens.is_cuda and seq_lens.dtype == torch.int32 and seq_lens.numel() >= B
             and seq_lens.is_contiguous(), "seq_lens must be contiguous cuda int32 [B]")
    W = block_table.shape[1]
    max_pages = W if max_pages is None else int(max_pages)
    _require(0 < max_pages <= W, "max_pages must be in [1, block_table width]")
    if out is None:
        out = torch.empty((B, HEADS_Q, HEAD_DIM), dtype=torch.float32, device=q.device)
    _require(out.dtype == torch.float32 and tuple(out.shape) == (B, HEADS_Q, HEAD_DIM) and out.stride(2) == 1
             and out.stride(1) % 2 == 0, "out must be fp32 [B, 32, 128] with contiguous dims")
    if lse is not None:
        _require(lse.dtype == torch.float32 and lse.is_contiguous() and lse.numel() >= B * HEADS_Q,
                 "lse must be contiguous fp32 [B, 32]")
    rc = lib().abkv_decode_attn_f32(_ptr(q), q.stride(0), q.stride(1), _ptr(kv_cache), kv_cache.shape[0],
                                    _ptr(block_table), _row_stride(block_table), _ptr(seq_lens), B, max_pages,
                                    float(scale), _ptr(out), out.stride(0), out.stride(1), _ptr(lse),
                                    C.c_void_p(_stream()))
    check(rc, "abkv_decode_attn_f32")
    return out, lse


def _layer_ptrs(layer_caches):
    _require(0 < len(layer_caches) <= 16, "between 1 and 16 layer caches per launch")
    for c in layer_caches:
        _check_cache(c)
    _require(len({c.shape[0] for c in layer_caches}) == 1, "layer caches of one launch must have equal page counts")
    arr = (C.c_void_p * len(layer_caches))(*[c.data_ptr() for c in layer_caches])
    return arr, layer_caches[0].shape[0]


def kv_move_segments(layer_caches, ops: torch.Tensor, seg_offsets: torch.Tensor) -> None:
    """Apply compaction copy ops (int32 [n, 4] on the GPU) to every layer cache, one workgroup per
    (segment, layer). See abkv_kv_move_segments for the ordering precondition inside a segment."""
    _require(ops.is_cuda and ops.dtype == torch.int32 and ops.dim() == 2 and ops.shape[1] == 4
             and ops.is_contiguous(), "ops must be contiguous cuda int32 [n, 4]")
    _require(seg_offsets.is_cuda and seg_offsets.dtype == torch.int32 and seg_offsets.is_contiguous(),
             "seg_offsets must be contiguous cuda int32")
    n_seg = seg_offsets.numel() - 1
    if n_seg <= 0 or ops.shape[0] == 0:
        return
    arr, num_pages = _layer_ptrs(layer_caches)
    rc = lib().abkv_kv_move_segments(arr, len(layer_caches), num_pages, PAGE, PAGE_BYTES, HALF_BYTES, SLOT_BYTES, _ptr(ops),
                                     _ptr(seg_offsets), n_seg, C.c_void_p(_stream()))
    check(rc, "abkv_kv_move_segments")


def kv_move_mixed(layer_caches, ops: torch.Tensor, seg_offsets: torch.Tensor, free_ops: torch.Tensor) -> None:
    """abkv_kv_move_mixed, one launch: the ordered segments of :func:`kv_move_segments` (``ops`` [n, 4] with
    ``seg_offsets`` [n_seg + 1]; n_seg may be 0) and the independent ops ``free_ops`` [m, 4] -- ops that read or write
    no slot another op of the call writes (:func:`abridgekv_amd.worker.pack_fused_moves` builds both)."""
    for name, t in (("ops", ops), ("free_ops", free_ops)):
        _require(t.is_cuda and t.dtype == torch.int32 and t.dim() == 2 and t.shape[1] == 4 and t.is_contiguous(),
                 f"{name} must be contiguous cuda int32 [n, 4]")
    _require(seg_offsets.is_cuda and seg_offsets.dtype == torch.int32 and seg_offsets.is_contiguous()
             and seg_offsets.numel() >= 1, "seg_offsets must be contiguous cuda int32 with at least one entry")
    n_seg = seg_offsets.numel() - 1 if ops.shape[0] else 0
    n_free = free_ops.shape[0]
    if n_seg == 0 and n_free == 0:
        return
    arr, num_pages = _layer_ptrs(layer_caches)
    rc = lib().abkv_kv_move_mixed(arr, len(layer_caches), num_pages, PAGE, PAGE_BYTES, HALF_BYTES, SLOT_BYTES,
                                  _ptr(ops) if n_seg else None, _ptr(seg_offsets) if n_seg else None, n_seg,
                                  _ptr(free_ops) if n_free else None, n_free, C.c_void_p(_stream()))
    check(rc, "abkv_kv_move_mixed")


def kv_copy_staged(layer_caches, ops: torch.Tensor, stage: torch.Tensor | None = None) -> None:
    """Gather-then-scatter for an arbitrary op list, staged through a workspace."""
    _require(ops.is_cuda and ops.dtype == torch.int32 and ops.dim() == 2 and ops.shape[1] == 4
             and ops.is_contiguous(), "ops must be contiguous cuda int32 [n, 4]")
    n = ops.shape[0]
    if n == 0:
        return
    arr, num_pages = _layer_ptrs(layer_caches)
    need = lib().abkv_kv_stage_bytes(len(layer_caches), n, SLOT_BYTES)
    if stage is None:
        stage = torch.empty(need, dtype=torch.uint8, device=ops.device)
    nbytes = stage.numel() * stage.element_size()
    _require(nbytes >= need, "stage buffer too small")
    rc = lib().abkv_kv_copy_staged(arr, len(layer_caches), num_pages, PAGE, PAGE_BYTES, HALF_BYTES, SLOT_BYTES, _ptr(ops), n,
                                   _ptr(stage), nbytes, C.c_void_p(_stream()))
    check(rc, "abkv_kv_copy_staged")


def kv_append(key: torch.Tensor, value: torch.Tensor, slot_mapping: torch.Tensor, kv_cache: torch.Tensor) -> None:
    """reshape_and_cache: write key/value [T, 8, 128] bf16 rows at slot_mapping [T] int64 (negative = skip)."""
    _check_cache(kv_cache)
    T = slot_mapping.numel()
    for name, t in (("key", key), ("value", value)):
        _require(t.is_cuda and t.dtype == torch.bfloat16 and t.shape[0] >= T
                 and tuple(t.shape[1:]) == (HEADS_KV, HEAD_DIM) and t.stride(2) == 1 and t.stride(1) == HEAD_DIM,
                 f"{name} must be cuda bf16 [T, {HEADS_KV}, {HEAD_DIM}] with contiguous rows")
    _require(slot_mapping.is_cuda and slot_mapping.dtype == torch.int64 and slot_mapping.is_contiguous(),
             "slot_mapping must be contiguous cuda int64")
    if T == 0:
        return
    rc = lib().abkv_kv_append(_ptr(key), key.stride(0) * 2, _ptr(value), value.stride(0) * 2, _ptr(slot_mapping), T,
                              _ptr(kv_cache), kv_cache.shape[0], PAGE_BYTES, HALF_BYTES, SLOT_BYTES, PAGE,
                              C.c_void_p(_stream()))
    check(rc, "abkv_kv_append")


def rope_cos_sin_cache(max_pos: int, theta: float = 1e6, device=None) -> torch.Tensor:
    """[max_pos, 128] fp32 table of cos then sin of the 64 NeoX rotary frequencies, computed as HF's default
    rotary embedding computes them (fp32 inverse frequencies theta^(-2i/128), fp32 products)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, HEAD_DIM, 2, dtype=torch.int64).float() / HEAD_DIM))
    freqs = torch.arange(max_pos, dtype=torch.float32)[:, None] * inv_freq[None, :]
    return torch.cat([freqs.cos(), freqs.sin()], dim=1).contiguous().to(device)


def rotary_cos_sin_from_model(rotary_emb, max_pos: int, device) -> torch.Tensor:
    """The same table from a HuggingFace rotary-embedding module (whatever its scaling), in fp32."""
    x = torch.zeros((1, 1, HEAD_DIM), dtype=torch.float32, device=device)
    cos, sin = rotary_emb(x, torch.arange(max_pos, device=device).view(1, -1))
    half = HEAD_DIM // 2
    return torch.cat([cos[0, :, :half], sin[0, :, :half]], dim=1).float().contiguous()


def rope_bound(max_position: int, block_c: int = 0, codes_k: int = 0) -> int:
    """Largest RoPE position of any token whose position (logical when block_c > 0) is <= max_position. In the
    abridged layout block b's content rows map to b*C + offset and its code rows to b*C + (an offset < C), so a token
    at logical (b, w) bounds every earlier token by b*C + min(w, C - 1)."""
    if not block_c:
        return int(max_position)
    blk, w = divmod(int(max_position), block_c + codes_k)
    return blk * block_c + min(w, block_c - 1)


def rope_kv_append(q: torch.Tensor, key: torch.Tensor, value: torch.Tensor, positions: torch.Tensor,
                   cos_sin: torch.Tensor, slot_mapping: torch.Tensor | None = None,
                   kv_cache: torch.Tensor | None = None, block_c: int = 0, codes_k: int = 0,
                   max_position: int | None = None, code_span: int = 0) -> None:
    """Rotate q [T, 32, 128] and key [T, 8, 128] in place (NeoX halves) and write rotated key and value rows at
    slot_mapping (int64, < 0 = skip; None = rotate only). positions [T] int64: RoPE positions, or logical positions
    of the abridged layout when block_c > 0 (mapped to bitrev RoPE positions on the device; codes_k a power of two
    <= block_c; the code rows spread over in-block offsets [0, code_span), 0 meaning block_c, block_c - T with a
    retained tail). ``max_position``: a host bound on ``positions`` (None: read back from the device, which
    synchronises); the RoPE positions it implies must lie inside ``cos_sin`` (ValueError otherwise)."""
    T = positions.numel()
    _require(q.is_cuda and q.dtype == torch.bfloat16 and q.dim() == 3 and tuple(q.shape[1:]) == (HEADS_Q, HEAD_DIM)
             and q.stride(2) == 1 and q.shape[0] >= T, "q must be cuda bf16 [T, 32, 128] with contiguous dims")
    for name, t in (("key", key), ("value", value)):
        _require(t.is_cuda and t.dtype == torch.bfloat16 and t.dim() == 3 and t.shape[0] >= T
                 and tuple(t.shape[1:]) == (HEADS_KV, HEAD_DIM) and t.stride(2) == 1 and t.stride(1) == HEAD_DIM,
                 f"{name} must be cuda bf16 [T, 8, 128] with contiguous rows")
    _require(positions.is_cuda and positions.dtype == torch.int64 and positions.is_contiguous(),
             "positions must be contiguous cuda int64")
    _require(cos_sin.is_cuda and cos_sin.dtype == torch.float32 and cos_sin.dim() == 2
             and cos_sin.shape[1] == HEAD_DIM and cos_sin.is_contiguous(), "cos_sin must be contiguous cuda fp32 [P, 128]")
    if block_c:
        _require(block_c > 0 and codes_k > 0 and codes_k & (codes_k - 1) == 0 and codes_k <= block_c,
                 "codes_k must be a power of two <= block_c")
        _require(code_span == 0 or codes_k <= code_span <= block_c, "code_span must be 0 or in [codes_k, block_c]")
    num_pages = 0
    if slot_mapping is not None:
        _check_cache(kv_cache)
        _require(slot_mapping.is_cuda and slot_mapping.dtype == torch.int64 and slot_mapping.is_contiguous()
                 and slot_mapping.numel() >= T, "slot_mapping must be contiguous cuda int64 [T]")
        num_pages = kv_cache.shape[0]
    if T == 0:
        return
    if max_position is None:
        max_position = int(positions.max())
    _require(rope_bound(max_position, block_c, codes_k) < cos_sin.shape[0],
             f"RoPE positions up to {rope_bound(max_position, block_c, codes_k)} exceed the cos/sin table "
             f"({cos_sin.shape[0]} rows)")
    rc = lib().abkv_rope_kv_append(_ptr(q), q.stride(0), q.stride(1), _ptr(key), key.stride(0), _ptr(value),
                                   value.stride(0), _ptr(positions), T, int(block_c), int(codes_k),
                                   int(code_span), _ptr(cos_sin), cos_sin.shape[0], _ptr(slot_mapping),
                                   _ptr(kv_cache), num_pages, C.c_void_p(_stream()))
    check(rc, "abkv_rope_kv_append")


def slot_mapping(req_idx: torch.Tensor, positions: torch.Tensor, block_table: torch.Tensor,
                 out: torch.Tensor | None = None, compacted: torch.Tensor | None = None) -> torch.Tensor:
    """Device slot mapping of one KV-cache group: table[req][p // 16] * 16 + p % 16 with p = positions -
    compacted[req] (``compacted`` [num_reqs] int32: tokens the group removed per request; None: positions are
    physical). Positions before the table or past its width map to -1."""
    _require(req_idx.is_cuda and req_idx.dtype == torch.int32 and req_idx.is_contiguous(), "req_idx: cuda int32")
    _require(positions.is_cuda and positions.dtype == torch.int64 and positions.is_contiguous(),
             "positions: cuda int64")
    _require(block_table.is_cuda and block_table.dtype == torch.int32 and block_table.is_contiguous(),
             "block_table: contiguous cuda int32 [B, W]")
    if compacted is not None:
        _require(compacted.is_cuda and compacted.dtype == torch.int32 and compacted.is_contiguous()
                 and compacted.numel() >= block_table.shape[0], "compacted: contiguous cuda int32 [num_reqs]")
    n = positions.numel()
    if out is None:
        out = torch.empty(n, dtype=torch.int64, device=positions.device)
    _require(req_idx.numel() == n, "req_idx and positions must have the same length")
    rc = lib().abkv_slot_mapping(_ptr(req_idx), _ptr(positions), n, _ptr(block_table), block_table.shape[0],
                                 block_table.shape[1], PAGE, _ptr(compacted), _ptr(out), C.c_void_p(_stream()))
    check(rc, "abkv_slot_mapping")
    return out


def prefill_masked_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_c: int, codes_k: int,
                             num_blocks: int, prompt_len: torch.Tensor | None = None,
                             head_quota: torch.Tensor | None = None, scale: float | None = None,
                             out: torch.Tensor | None = None, lse: torch.Tensor | None = None, retain_tail: int = 0,
                             tail_policy: str = "static", pause_xattn: str = "full", pause_passes: int = 1,
                             copy_rows: int = 0, replay_rows: int = 0, replay_exclude: bool = False):
    """Teacher-forced attention under the compression mask (N blocks of [C content | L passes of K codes],
    L = ``pause_passes``: pass l reads its block's content, its pass l - 1 and its own pass by ``pause_xattn``; later
    blocks read the final pass only; L > 1 evaluates the mask per element), ``replay_rows`` = R replay rows after each
    block's codes (a block's last R content tokens again: they see their block and its final pass; content row i of
    the next block sees them from row i on; ``replay_exclude`` hides the last R content rows from the codes), then
    ``copy_rows`` rows of a copy region that see the last block's final pass and themselves causally. ``codes_k`` = 0:
    causal attention within blocks of C rows (the plain forward).

    q [B, S0, 32, 128], k/v [B, S0, 8, 128] bf16 (any strides with contiguous dims, e.g. the [B, H, S, D]
    transposed views HF attention receives, permuted back); prompt_len [B] int32 raw-prompt content tokens;
    head_quota [32] int32 code slots visible per query head; retain_tail = T of a retained tail (a block's last T
    content rows, hidden from its own codes) and ``tail_policy`` the later rows that see it: "static" every later row,
    "sticky" the next block's content rows, "rolling" the next block's i-th content row from tail row i on, "raw"
    (CompressLM's raw_tail, T <= C) as rolling but not hidden from the codes;
    ``pause_xattn`` a code row's attention to its block's code rows ("full", "causal", "none"; the non-full ones
    evaluate the mask per element). Returns
    (out [B, S0, 32, 128] bf16, lse [B, 32, S0] fp32 natural log or None). fp32 q/k/v select the fp32 mode (out fp32).
    """
    B, S0 = q.shape[0], q.shape[1]
    policy = _tail(block_c, retain_tail, tail_policy)
    xattn = xattn_code(pause_xattn)
    L, cr = _passes(pause_passes), _copy_rows(codes_k, pause_passes, copy_rows)
    R, rx = _replay(block_c, codes_k, retain_tail, replay_rows, replay_exclude)
    if q.dtype == torch.float32:
        return _prefill_masked_f32(q, k, v, block_c, codes_k, num_blocks, prompt_len, head_quota, scale, out, lse,
                                   int(retain_tail), policy, xattn, L, cr, R, rx)
    _require(S0 == num_blocks * (block_c + L * codes_k + R) + cr,
             "seq_len must be num_blocks * (block_c + L * codes_k + replay_rows) + copy_rows")
    for name, t, h in (("q", q, HEADS_Q), ("k", k, HEADS_KV), ("v", v, HEADS_KV)):
        _require(t.is_cuda and t.dtype == torch.bfloat16 and t.dim() == 4 and tuple(t.shape) == (B, S0, h, HEAD_DIM)
                 and t.stride(3) == 1, f"{name} must be cuda bf16 [B, S0, {h}, {HEAD_DIM}] with contiguous dims")
    if prompt_len is not None:
        _require(prompt_len.is_cuda and prompt_len.dtype == torch.int32 and prompt_len.numel() == B
                 and prompt_len.is_contiguous(), "prompt_len must be contiguous cuda int32 [B]")
    if head_quota is not None:
        _require(head_quota.is_cuda and head_quota.dtype == torch.int32 and head_quota.numel() == HEADS_Q
                 and head_quota.is_contiguous(), "head_quota must be contiguous cuda int32 [32]")
    if out is None:
        out = torch.empty((B, S0, HEADS_Q, HEAD_DIM), dtype=torch.bfloat16, device=q.device)
    _require(out.dtype == torch.bfloat16 and tuple(out.shape) == (B, S0, HEADS_Q, HEAD_DIM) and out.stride(3) == 1,
             "out must be bf16 [B, S0, 32, 128] with contiguous dims")
    if lse is not None:
        _require(lse.dtype == torch.float32 and lse.is_contiguous() and tuple(lse.shape) == (B, HEADS_Q, S0),
                 "lse must be contiguous fp32 [B, 32, S0]")
    scale = default_scale() if scale is None else float(scale)
    rc = lib().abkv_prefill_masked_attn(_ptr(q), q.stride(0), q.stride(1), q.stride(2), _ptr(k), k.stride(0),
                                        k.stride(1), k.stride(2), _ptr(v), v.stride(0), v.stride(1), v.stride(2), B,
                                        block_c, codes_k, num_blocks, S0, _ptr(prompt_len), _ptr(head_quota),
                                        int(retain_tail), policy, xattn, L, cr, R, rx, scale, _ptr(out),
                                        out.stride(0),
                                        out.stride(1), out.stride(2), _ptr(lse), C.c_void_p(_stream()))
    check(rc, "abkv_prefill_masked_attn")
    return out, lse


def prefill_masked_attention_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                                      lse: torch.Tensor, dout: torch.Tensor, block_c: int, codes_k: int,
                                      num_blocks: int, prompt_len: torch.Tensor | None = None,
                                      head_quota: torch.Tensor | None = None, scale: float | None = None,
                                      retain_tail: int = 0, tail_policy: str = "static", pause_xattn: str = "full",
                                      pause_passes: int = 1, copy_rows: int = 0, replay_rows: int = 0,
                                      replay_exclude: bool = False):
    """Gradients (dq [B, S0, 32, 128], dk, dv [B, S0, 8, 128], bf16) of sum(dout * out) for
    :func:`prefill_masked_attention` under the same mask, from its out and lse (bf16 path only)."""
    B, S0 = q.shape[0], q.shape[1]
    policy = _tail(block_c, retain_tail, tail_policy)
    xattn = xattn_code(pause_xattn)
    L, cr = _passes(pause_passes), _copy_rows(codes_k, pause_passes, copy_rows)
    R, rx = _replay(block_c, codes_k, retain_tail, replay_rows, replay_exclude)
    _require(S0 == num_blocks * (block_c + L * codes_k + R) + cr,
             "seq_len must be num_blocks * (block_c + L * codes_k + replay_rows) + copy_rows")
    for name, t, h in (("q", q, HEADS_Q), ("k", k, HEADS_KV), ("v", v, HEADS_KV), ("out", out, HEADS_Q),
                       ("dout", dout, HEADS_Q)):
        _require(t.is_cuda and t.dtype == torch.bfloat16 and t.dim() == 4 and tuple(t.shape) == (B, S0, h, HEAD_DIM)
                 and t.stride(3) == 1, f"{name} must be cuda bf16 [B, S0, {h}, {HEAD_DIM}] with contiguous dims")
    _require(lse.is_cuda and lse.dtype == torch.float32 and lse.is_contiguous()
             and tuple(lse.shape) == (B, HEADS_Q, S0), "lse must be contiguous cuda fp32 [B, 32, S0]")
    if prompt_len is not None:
        _require(prompt_len.is_cuda and prompt_len.dtype == torch.int32 and prompt_len.numel() == B
                 and prompt_len.is_contiguous(), "prompt_len must be contiguous cuda int32 [B]")
    if head_quota is not None:
        _require(head_quota.is_cuda and head_quota.dtype == torch.int32 and head_quota.numel() == HEADS_Q
                 and head_quota.is_contiguous(), "head_quota must be contiguous cuda int32 [32]")
    scale = default_scale() if scale is None else float(scale)
    dq = torch.empty((B, S0, HEADS_Q, HEAD_DIM), dtype=torch.bfloat16, device=q.device)
    dk = torch.empty((B, S0, HEADS_KV, HEAD_DIM), dtype=torch.bfloat16, device=q.device)
    dv = torch.empty_like(dk)
    ws = torch.empty(lib().abkv_prefill_masked_bwd_workspace_size(B, S0), dtype=torch.uint8, device=q.device)
    args = []
    for t in (q, k, v, out, dout):
        args += [_ptr(t), t.stride(0), t.stride(1), t.stride(2)]
    args += [_ptr(lse), B, block_c, codes_k, num_blocks, S0, _ptr(prompt_len), _ptr(head_quota), int(retain_tail),
             policy, xattn, L, cr, R, rx, scale]
    for t in (dq, dk, dv):
        args += [_ptr(t), t.stride(0), t.stride(1), t.stride(2)]
    rc = lib().abkv_prefill_masked_attn_bwd(*args, _ptr(ws), ws.numel(), C.c_void_p(_stream()))
    check(rc, "abkv_prefill_masked_attn_bwd")
    return dq, dk, dv


TAIL_POLICIES = ("static", "rolling", "sticky", "raw")     # the kernels' policy codes 0, 1, 2, 3


def tail_policy_code(tail_policy: str) -> int:
    """Kernel code of a retain_tail_policy name ("raw": CompressLM's raw_tail, the rolling window that the codes also
    see)."""
    _require(tail_policy in TAIL_POLICIES, f"tail_policy must be one of {TAIL_POLICIES}, got {tail_policy!r}")
    return TAIL_POLICIES.index(tail_policy)


def _tail(block_c: int, retain_tail: int, tail_policy: str) -> int:
    """Checks the tail size for its policy (a raw tail may span the whole block, compress_forward.py:270-271) and
    returns the policy's kernel code."""
    policy = tail_policy_code(tail_policy)
    if tail_policy == "raw":
        _require(0 <= int(retain_tail) <= block_c, "a raw tail must be in [0, block_c]")
    else:
        _require(0 <= int(retain_tail) < block_c, "retain_tail must be in [0, block_c)")
    return policy


XATTN = ("full", "causal", "none")                  # the kernels' pause_xattn codes 0, 1, 2


def xattn_code(pause_xattn: str) -> int:
    """Kernel code of a pause_xattn name."""
    _require(pause_xattn in XATTN, f"pause_xattn must be one of {XATTN}, got {pause_xattn!r}")
    return XATTN.index(pause_xattn)


def _passes(pause_passes) -> int:
    _require(int(pause_passes) == pause_passes and int(pause_passes) >= 1, "pause_passes must be an integer >= 1")
    return int(pause_passes)


def _replay(block_c, codes_k, retain_tail, replay_rows, replay_exclude) -> tuple[int, int]:
    R = int(replay_rows)
    _require(0 <= R <= block_c and R == replay_rows, "replay_rows must be an integer in [0, block_c]")
    _require(not (R and (retain_tail or codes_k == 0)), "replay rows need code rows and exclude a retained tail")
    _require(not replay_exclude or 0 < R < block_c, "replay_exclude requires replay_rows in [1, block_c)")
    return R, int(bool(replay_exclude))


def _copy_rows(codes_k, pause_passes, copy_rows) -> int:
    _require(int(codes_k) >= 0, "codes_k must be >= 0")
    _require(int(copy_rows) == copy_rows and int(copy_rows) >= 0, "copy_rows must be an integer >= 0")
    _require(codes_k > 0 or (pause_passes == 1 and copy_rows == 0),
             "codes_k = 0 (plain causal attention) takes one pass and no copy rows")
    return int(copy_rows)


def _prefill_masked_f32(q, k, v, block_c, codes_k, num_blocks, prompt_len, head_quota, scale, out, lse, retain_tail,
                        policy, xattn, passes, copy_rows, replay_rows=0, replay_exclude=0):
    B, S0 = q.shape[0], q.shape[1]
    _require(S0 == num_blocks * (block_c + passes * codes_k + replay_rows) + copy_rows,
             "seq_len must be num_blocks * (block_c + L * codes_k + replay_rows) + copy_rows")
    for name, t, h in (("q", q, HEADS_Q), ("k", k, HEADS_KV), ("v", v, HEADS_KV)):
        _require(t.is_cuda and t.dtype == torch.float32 and t.dim() == 4 and tuple(t.shape) == (B, S0, h, HEAD_DIM)
                 and t.stride(3) == 1 and all(x % 4 == 0 for x in t.stride()[:3]),
                 f"{name} must be cuda fp32 [B, S0, {h}, {HEAD_DIM}] with contiguous, 16-byte aligned rows")
    if prompt_len is not None:
        _require(prompt_len.is_cuda and prompt_len.dtype == torch.int32 and prompt_len.numel() == B
                 and prompt_len.is_contiguous(), "prompt_len must be contiguous cuda int32 [B]")
    if head_quota is not None:
        _require(head_quota.is_cuda and head_quota.dtype == torch.int32 and head_quota.numel() == HEADS_Q
                 and head_quota.is_contiguous(), "head_quota must be contiguous cuda int32 [32]")
    if out is None:
        out = torch.empty((B, S0, HEADS_Q, HEAD_DIM), dtype=torch.float32, device=q.device)
    _require(out.dtype == torch.float32 and tuple(out.shape) == (B, S0, HEADS_Q, HEAD_DIM) and out.stride(3) == 1
             and all(x % 2 == 0 for x in out.stride()[:3]), "out must be fp32 [B, S0, 32, 128] with contiguous dims")
    if lse is not None:
        _require(lse.dtype == torch.float32 and lse.is_contiguous() and tuple(lse.shape) == (B, HEADS_Q, S0),
                 "lse must be contiguous fp32 [B, 32, S0]")
    scale = default_scale() if scale is None else float(scale)
    rc = lib().abkv_prefill_masked_attn_f32(_ptr(q), q.stride(0), q.stride(1), q.stride(2), _ptr(k), k.stride(0),
                                            k.stride(1), k.stride(2), _ptr(v), v.stride(0), v.stride(1), v.stride(2),
                                            B, block_c, codes_k, num_blocks, S0, _ptr(prompt_len), _ptr(head_quota),
                                            retain_tail, policy, xattn, passes, copy_rows, replay_rows,
                                            replay_exclude, scale, _ptr(out),
                                            out.stride(0),
                                            out.stride(1), out.stride(2), _ptr(lse), C.c_void_p(_stream()))
    check(rc, "abkv_prefill_masked_attn_f32")
    return out, lse


def paged_split_plan(num_tiles: int, max_keys: int, target_blocks: int | None = None, min_split_tiles: int = 8):
    """(num_splits, split_tiles) for a paged multi-query launch of num_tiles query tiles whose longest key range is
    max_keys: split along the keys only when the 8 KV heads x num_tiles workgroups cannot fill the GPU, into as many
    splits as one round of workgroups holds (the kernel runs one workgroup per CU: target_blocks = the CU count).
    A code step of one request (32 workgroups) over 5000 / 12000 keys: 8 splits 47 / 75 us with the merge, 9-10
    splits (two rounds) 63 / 108 us, 16 splits 67 / 94 us."""
    max_kt = -(-int(max_keys) // 64)
    blocks = num_tiles * HEADS_KV
    target = _num_cus() if target_blocks is None else int(target_blocks)
    n = min(target // blocks, max_kt // min_split_tiles)
    if n < 2:
        return 1, 0
    split_tiles = -(-max_kt // n)
    return -(-max_kt // split_tiles), split_tiles


def _excluded_pairs(excluded, B):
    """Per-request excluded key ranges as int32 [B, 2] (an empty range for None entries), or None for none at all."""
    import numpy as np

    if excluded is None:
        return None
    ex = list(excluded)
    _require(len(ex) == B, "excluded: one (start, end) or None per request")
    pairs = np.zeros((B, 2), dtype=np.int64)
    for r, e in enumerate(ex):
        if e is not None:
            s, t = int(e[0]), int(e[1])
            _require(0 <= s <= t, "excluded ranges must satisfy 0 <= start <= end")
            pairs[r] = (s, t)
    return pairs if pairs[:, 1].max(initial=0) > 0 else None


def paged_prefill_attention(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor, q_start, kv_start,
                            kv_limit, causal, scale: float | None = None, out: torch.Tensor | None = None,
                            lse: torch.Tensor | None = None, split: int | None = None, excluded=None):
    """Multi-query attention over the paged cache (prompt chunks: causal; CompressLM code step: non-causal with
    kv_limit = physical code start + quota).

    q [T, 32, 128] bf16; block_table [B, W] int32 on the GPU; q_start [B+1], kv_start [B], kv_limit [B]: host
    sequences (the metadata builder's CPU copies) -- request r's queries are tokens q_start[r]..q_start[r+1]-1 at
    physical positions kv_start[r] + i, seeing keys < kv_limit[r] (and <= their own position when causal).
    ``causal``: a bool for the whole batch or one flag per request (code steps and prompt chunks may share a batch).
    ``excluded``: None, or per request a physical (start, end) its queries must not see (None: nothing), e.g. the
    code step's own-block retained tail. ``split``: key splits (None: chosen by :func:`paged_split_plan`; 1: no split).
    Returns (out [T, 32, 128] bf16, lse [T, 32] fp32 or None). fp32 q and cache select the fp32 mode (out fp32).
    """
    import numpy as np

    f32 = q.dtype == torch.float32
    dt = torch.float32 if f32 else torch.bfloat16
    _check_cache(kv_cache, dt)
    _require(q.is_cuda and q.dtype == dt and q.dim() == 3 and tuple(q.shape[1:]) == (HEADS_Q, HEAD_DIM)
             and q.stride(2) == 1, "q must be cuda [T, 32, 128] with contiguous dims")
    _require(block_table.is_cuda and block_table.dtype == torch.int32 and block_table.dim() == 2
             and block_table.stride(1) == 1, "block_table must be cuda int32 [B, W]")
    qs = np.asarray(q_start, dtype=np.int64)
    ks = np.asarray(kv_start, dtype=np.int64)
    kl = np.asarray(kv_limit, dtype=np.int64)
    B = ks.size
    W = block_table.shape[1]
    _require(qs.size == B + 1 and kl.size == B and B <= block_table.shape[0], "q_start [B+1], kv_start/kv_limit [B]")
    _require(qs[0] == 0 and np.all(np.diff(qs) >= 0) and qs[-1] <= q.shape[0], "q_start must be a prefix sum <= T")
    _require(np.all(kl >= 0) and np.all(kl <= W * PAGE), "kv_limit must lie in [0, block_table width * 16]")
    _require(np.all(ks >= 0), "kv_start must be non-negative")
    T = q.shape[0]
    if out is None:
        out = torch.empty((T, HEADS_Q, HEAD_DIM), dtype=dt, device=q.device)
    _require(out.dtype == dt and tuple(out.shape) == (T, HEADS_Q, HEAD_DIM) and out.stride(2) == 1,
             "out must be [T, 32, 128] (dtype of q) with contiguous dims")
    if lse is not None:
        _require(lse.dtype == torch.float32 and lse.is_contiguous() and tuple(lse.shape) == (T, HEADS_Q),
                 "lse must be contiguous fp32 [T, 32]")
    nq = np.diff(qs)
    exd = _excluded_pairs(excluded, B)
    ex_t = None if exd is None else torch.from_numpy(exd.astype(np.int32).reshape(-1)).to(q.device)
    if f32:
        if qs[-1] == 0:
            return out, lse
        dev = q.device
        cz = np.broadcast_to(np.asarray(causal, dtype=np.int64), (B,)).astype(np.int64)
        tok_req = np.repeat(np.arange(B), nq)
        meta = torch.from_numpy(np.concatenate([qs, ks, kl, cz, tok_req]).astype(np.int32)).to(dev)
        o1, o2, o3, o4 = B + 1, 2 * B + 1, 3 * B + 1, 4 * B + 1
        scale = default_scale() if scale is None else float(scale)
        rc = lib().abkv_paged_prefill_attn_f32(_ptr(q), q.stride(0), q.stride(1), _ptr(kv_cache), kv_cache.shape[0],
                                               _ptr(block_table), _row_stride(block_table), W, _ptr(meta[:o1]),
                                               _ptr(meta[o1:o2]), _ptr(meta[o2:o3]), _ptr(ex_t), _ptr(meta[o4:]),
                                               int(qs[-1]), _ptr(meta[o3:o4]), 1, scale, _ptr(out), out.stride(0),
                                               out.stride(1), _ptr(lse), C.c_void_p(_stream()))
        check(rc, "abkv_paged_prefill_attn_f32")
        return out, lse
    tiles = [(r, q0) for r in range(B) for q0 in range(0, int(nq[r]), 64)]
    if not tiles:
        return out, lse
    tr = np.asarray(tiles, dtype=np.int32)
    dev = q.device
    cz = np.broadcast_to(np.asarray(causal, dtype=np.int64), (B,)).astype(np.int64)
    meta = torch.from_numpy(np.concatenate([qs, ks, kl, cz]).astype(np.int32)).to(dev)
    tl = torch.from_numpy(np.ascontiguousarray(tr.T)).to(dev)
    q_start_d, kv_start_d = meta[: B + 1], meta[B + 1: 2 * B + 1]
    kv_limit_d, causal_d = meta[2 * B + 1: 3 * B + 1], meta[3 * B + 1:]
    scale = default_scale() if scale is None else float(scale)
    max_keys = int(kl.max()) if kl.size else 0
    if split is None:
        n_splits, split_tiles = paged_split_plan(len(tiles), max_keys)
    else:
        n_splits = max(1, int(split))
        split_tiles = -(-(-(-max_keys // 64)) // n_splits) if n_splits > 1 else 0
    ws, ws_bytes = None, 0
    covered = int(qs[-1])                    # rows the launch writes; rows past q_start[-1] stay untouched
    if n_splits > 1:
        _require(n_splits * split_tiles * 64 >= max_keys, "key splits must cover every key")
        ws_bytes = lib().abkv_paged_prefill_workspace_size(covered, n_splits)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    rc = lib().abkv_paged_prefill_attn(_ptr(q), q.stride(0), q.stride(1), _ptr(kv_cache), kv_cache.shape[0],
                                       _ptr(block_table), _row_stride(block_table), W, _ptr(q_start_d),
                                       _ptr(kv_start_d), _ptr(kv_limit_d), _ptr(ex_t), _ptr(tl[0]), _ptr(tl[1]),
                                       len(tiles),
                                       _ptr(causal_d), 1, scale, _ptr(out), out.stride(0), out.stride(1), _ptr(lse),
                                       covered, n_splits, split_tiles, _ptr(ws), ws_bytes, C.c_void_p(_stream()))
    check(rc, "abkv_paged_prefill_attn")
    return out, lse


def _host_quota(head_quota):
    hq = [int(x) for x in head_quota]
    _require(len(hq) == HEADS_KV and all(1 <= x <= 2048 for x in hq), "head_quota must be 8 ints in [1, 2048]")
    return hq, (C.c_int32 * HEADS_KV)(*hq)


def _check_pool(pool: torch.Tensor, rows: int) -> None:
    _require(pool.is_cuda and pool.dtype == torch.bfloat16 and pool.dim() == 4 and pool.shape[1] == 2
             and pool.shape[2] == rows and pool.shape[3] == HEAD_DIM and pool.is_contiguous(),
             f"packed pool must be contiguous cuda bf16 [pages, 2, {rows}, {HEAD_DIM}]")


def _check_side_table(packed_table: torch.Tensor, packed_count: torch.Tensor, B: int) -> None:
    _require(packed_table.is_cuda and packed_table.dtype == torch.int32 and packed_table.dim() == 2
             and packed_table.shape[0] >= B and packed_table.stride(1) == 1,
             "packed_table must be cuda int32 [B, S] with contiguous rows")
    _require(packed_count.is_cuda and packed_count.dtype == torch.int32 and packed_count.numel() >= B
             and packed_count.is_contiguous(), "packed_count must be contiguous cuda int32 [B]")


def packed_capture(layer_caches, layer_pools, layer_rows: torch.Tensor, layer_quota: torch.Tensor,
                   block_table: torch.Tensor, code_start: torch.Tensor, dst_page: torch.Tensor) -> None:
    """Copy closed blocks' code rows into per-head packed pages, all layers in one launch.

    layer_caches / layer_pools: per layer the paged cache [P, 2, 16, 8, 128] and the packed pool
    [pool_pages, 2, rows_l, 128] (bf16); layer_rows [L] / layer_quota [L, 8]: cuda int32 (rows_l = sum of the row);
    block_table [n, W] cuda int32: the page table row of each capture's sequence; code_start / dst_page [n] cuda int32.
    """
    L = len(layer_caches)
    _require(L > 0 and len(layer_pools) == L, "one pool per layer cache")
    for c in layer_caches:
        _check_cache(c)
    _require(len({c.shape[0] for c in layer_caches}) == 1, "layer caches must have equal page counts")
    _require(len({p.shape[0] for p in layer_pools}) == 1, "layer pools must have equal page counts")
    _require(layer_rows.is_cuda and layer_rows.dtype == torch.int32 and layer_rows.numel() == L
             and layer_rows.is_contiguous(), "layer_rows must be contiguous cuda int32 [L]")
    _require(layer_quota.is_cuda and layer_quota.dtype == torch.int32 and tuple(layer_quota.shape) == (L, HEADS_KV)
             and layer_quota.is_contiguous(), "layer_quota must be contiguous cuda int32 [L, 8]")
    rows_host = layer_rows.cpu().tolist()
    for pool, rows in zip(layer_pools, rows_host):
        _check_pool(pool, int(rows))
    n = int(code_start.numel())
    _require(block_table.is_cuda and block_table.dtype == torch.int32 and block_table.dim() == 2
             and block_table.shape[0] >= n and block_table.stride(1) == 1, "block_table must be cuda int32 [n, W]")
    _require(code_start.is_cuda and code_start.dtype == torch.int32 and code_start.is_contiguous()
             and dst_page.is_cuda and dst_page.dtype == torch.int32 and dst_page.numel() == n
             and dst_page.is_contiguous(), "code_start / dst_page must be contiguous cuda int32 [n]")
    if n == 0:
        return
    dev = code_start.device
    ptrs = torch.tensor([c.data_ptr() for c in layer_caches] + [p.data_ptr() for p in layer_pools],
                        dtype=torch.int64).to(dev)
    rc = lib().abkv_packed_capture(_ptr(ptrs[:L]), _ptr(ptrs[L:]), _ptr(layer_rows), _ptr(layer_quota), L,
                                   layer_caches[0].shape[0], layer_pools[0].shape[0], _ptr(block_table),
                                   _row_stride(block_table), block_table.shape[1], _ptr(code_start), _ptr(dst_page),
                                   n, C.c_void_p(_stream()))
    check(rc, "abkv_packed_capture")


def decode_attention_packed(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor,
                            seq_lens: torch.Tensor, packed_pool: torch.Tensor, head_quota, packed_table: torch.Tensor,
                            packed_count: torch.Tensor, scale: float, max_pages: int | None = None,
                            max_packed: int | None = None, out: torch.Tensor | None = None,
                            lse: torch.Tensor | None = None, split_pages: int = DEFAULT_SPLIT_PAGES,
                            workspace: torch.Tensor | None = None):
    """Decode attention of one layer over the paged rows plus each sequence's per-head packed code pages.

    As :func:`decode_attention`, plus packed_pool [pool_pages, 2, rows, 128] bf16 (this layer), head_quota (8 ints,
    this layer's quotas, rows = their sum), packed_table [B, S] / packed_count [B] cuda int32 (the sequences' packed
    page ids); ``max_packed`` bounds packed_count (defaults to S). Returns (out, lse).
    """
    _check_cache(kv_cache)
    _require(q.is_cuda and q.dtype == torch.bfloat16 and q.dim() == 3 and tuple(q.shape[1:]) == (HEADS_Q, HEAD_DIM)
             and q.stride(2) == 1, f"q must be cuda bf16 [B, {HEADS_Q}, {HEAD_DIM}] with contiguous dims")
    B = q.shape[0]
    _require(block_table.is_cuda and block_table.dtype == torch.int32 and block_table.dim() == 2
             and block_table.shape[0] >= B and block_table.stride(1) == 1, "block_table must be cuda int32 [B, W]")
    _require(seq_lens.is_cuda and seq_lens.dtype == torch.int32 and seq_lens.numel() >= B
             and seq_lens.is_contiguous(), "seq_lens must be contiguous cuda int32 [B]")
    _require(0 < split_pages <= 64 and split_pages % 2 == 0, "split_pages must be an even number in [2, 64]")
    hq, hq_c = _host_quota(head_quota)
    rows = sum(hq)
    _check_pool(packed_pool, rows)
    _check_side_table(packed_table, packed_count, B)
    W = block_table.shape[1]
    max_pages = W if max_pages is None else int(max_pages)
    _require(0 < max_pages <= W, "max_pages must be in [1, block_table width]")
    S = packed_table.shape[1]
    max_packed = S if max_packed is None else int(max_packed)
    _require(0 <= max_packed <= S and max_packed * max(hq) < (1 << 21), "max_packed must be in [0, packed_table width]")
    if out is None:
        out = torch.empty((B, HEADS_Q, HEAD_DIM), dtype=torch.bfloat16, device=q.device)
    _require(out.dtype == torch.bfloat16 and tuple(out.shape) == (B, HEADS_Q, HEAD_DIM) and out.stride(2) == 1,
             "out must be bf16 [B, 32, 128] with contiguous dims")
    if lse is not None:
        _require(lse.dtype == torch.float32 and lse.is_contiguous() and lse.numel() >= B * HEADS_Q,
                 "lse must be contiguous fp32 [B, 32]")
    sr = lib().abkv_decode_side_split_rows(min(hq))
    need = lib().abkv_decode_packed_workspace_size(B, max_pages, split_pages, max_packed, max(hq), sr)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_bytes = workspace.numel() * workspace.element_size()
    _require(ws_bytes >= need, "packed decode workspace too small")
    rc = lib().abkv_decode_attn_packed(_ptr(q), q.stride(0), q.stride(1), _ptr(kv_cache), kv_cache.shape[0],
                                       _ptr(block_table), _row_stride(block_table), _ptr(seq_lens), B, max_pages,
                                       split_pages, _ptr(packed_pool), packed_pool.shape[0], rows, hq_c,
                                       _ptr(packed_table), _row_stride(packed_table), _ptr(packed_count), max_packed,
                                       sr, float(scale), _ptr(out), out.stride(0), out.stride(1), _ptr(lse),
                                       _ptr(workspace), ws_bytes, C.c_void_p(_stream()))
    check(rc, "abkv_decode_attn_packed")
    return out, lse


def paged_prefill_attention_packed(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor, q_start,
                                   kv_start, kv_limit, causal, packed_pool: torch.Tensor, head_quota,
                                   packed_table: torch.Tensor, packed_count: torch.Tensor, max_packed: int,
                                   scale: float | None = None, out: torch.Tensor | None = None,
                                   lse: torch.Tensor | None = None, head_quota_dev: torch.Tensor | None = None,
                                   excluded=None):
    """Multi-query attention over the paged rows plus each request's per-head packed code pages (visible to every
    query). As :func:`paged_prefill_attention`; a non-causal request (code step) sees paged keys
    ``< min(kv_limit, kv_start + q_h)`` for KV head h, except its ``excluded`` range. ``max_packed`` bounds
    packed_count (<= 2048). Returns (out, lse).
    """
    import numpy as np

    _check_cache(kv_cache)
    _require(q.is_cuda and q.dtype == torch.bfloat16 and q.dim() == 3 and tuple(q.shape[1:]) == (HEADS_Q, HEAD_DIM)
             and q.stride(2) == 1, "q must be cuda bf16 [T, 32, 128] with contiguous dims")
    _require(block_table.is_cuda and block_table.dtype == torch.int32 and block_table.dim() == 2
             and block_table.stride(1) == 1, "block_table must be cuda int32 [B, W]")
    qs = np.asarray(q_start, dtype=np.int64)
    ks = np.asarray(kv_start, dtype=np.int64)
    kl = np.asarray(kv_limit, dtype=np.int64)
    B = ks.size
    W = block_table.shape[1]
    _require(qs.size == B + 1 and kl.size == B and B <= block_table.shape[0], "q_start [B+1], kv_start/kv_limit [B]")
    _require(qs[0] == 0 and np.all(np.diff(qs) >= 0) and qs[-1] <= q.shape[0], "q_start must be a prefix sum <= T")
    _require(np.all(kl >= 0) and np.all(kl <= W * PAGE) and np.all(ks >= 0), "kv ranges out of the table")
    hq, hq_c = _host_quota(head_quota)
    rows = sum(hq)
    _check_pool(packed_pool, rows)
    _check_side_table(packed_table, packed_count, B)
    max_packed = int(max_packed)
    _require(0 <= max_packed <= min(2048, packed_table.shape[1]) and max_packed * max(hq) < (1 << 21),
             "max_packed must be in [0, min(2048, packed_table width)]")
    T = q.shape[0]
    if out is None:
        out = torch.empty((T, HEADS_Q, HEAD_DIM), dtype=torch.bfloat16, device=q.device)
    _require(out.dtype == torch.bfloat16 and tuple(out.shape) == (T, HEADS_Q, HEAD_DIM) and out.stride(2) == 1,
             "out must be bf16 [T, 32, 128] with contiguous dims")
    if lse is not None:
        _require(lse.dtype == torch.float32 and lse.is_contiguous() and tuple(lse.shape) == (T, HEADS_Q),
                 "lse must be contiguous fp32 [T, 32]")
    nq = np.diff(qs)
    tiles = [(r, q0) for r in range(B) for q0 in range(0, int(nq[r]), 64)]
    if not tiles:
        return out, lse
    dev = q.device
    tr = np.asarray(tiles, dtype=np.int32)
    cz = np.broadcast_to(np.asarray(causal, dtype=np.int64), (B,)).astype(np.int64)
    meta = torch.from_numpy(np.concatenate([qs, ks, kl, cz, hq]).astype(np.int32)).to(dev)
    exd = _excluded_pairs(excluded, B)
    ex_t = None if exd is None else torch.from_numpy(exd.astype(np.int32).reshape(-1)).to(dev)
    tl = torch.from_numpy(np.ascontiguousarray(tr.T)).to(dev)
    o1, o2, o3, o4 = B + 1, 2 * B + 1, 3 * B + 1, 4 * B + 1
    if head_quota_dev is None:
        head_quota_dev = meta[o4:]
    _require(head_quota_dev.is_cuda and head_quota_dev.dtype == torch.int32 and head_quota_dev.numel() == HEADS_KV,
             "head_quota_dev must be cuda int32 [8]")
    scale = default_scale() if scale is None else float(scale)
    max_keys = int(kl.max()) if kl.size else 0
    n_splits, split_tiles = paged_split_plan(len(tiles), max_keys)
    if n_splits <= 1:
        n_splits, split_tiles = 1, max(1, -(-max_keys // 64))
    side_rows = max(1, max_packed * max(hq))
    side_tiles_all = -(-side_rows // 64)
    side_splits, side_split_tiles = paged_split_plan(len(tiles), side_rows)
    if side_splits <= 1:
        side_splits, side_split_tiles = 1, side_tiles_all
    covered = int(qs[-1])                    # rows the launch writes; rows past q_start[-1] stay untouched
    ws_bytes = lib().abkv_paged_prefill_workspace_size(covered, n_splits + side_splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    rc = lib().abkv_paged_prefill_attn_packed(
        _ptr(q), q.stride(0), q.stride(1), _ptr(kv_cache), kv_cache.shape[0], _ptr(block_table),
        _row_stride(block_table), W, _ptr(meta[:o1]), _ptr(meta[o1:o2]), _ptr(meta[o2:o3]), _ptr(ex_t), _ptr(tl[0]),
        _ptr(tl[1]), len(tiles), _ptr(meta[o3:o4]), 1, _ptr(head_quota_dev), _ptr(packed_pool), packed_pool.shape[0], rows, hq_c,
        _ptr(packed_table), _row_stride(packed_table), _ptr(packed_count), max_packed, scale, _ptr(out),
        out.stride(0), out.stride(1), _ptr(lse), covered, n_splits, split_tiles, side_splits, side_split_tiles, _ptr(ws),
        ws_bytes, C.c_void_p(_stream()))
    check(rc, "abkv_paged_prefill_attn_packed")
    return out, lse


def default_scale() -> float:
    return 1.0 / math.sqrt(HEAD_DIM)
