"""The kernels as torch custom ops (namespace ``abridgekv``), so compiled callers and captured graphs can hold them.

The reference reaches its attention kernels through torch ops of the serving stack (vLLM's registered attention /
``reshape_and_cache`` ops, FlashInfer's wrappers; the backend contract of
third_party/vllm_overlay/vllm/v1/worker/gpu_model_runner.py:1872-1887, 2184-2276). These registrations give this
library's kernels the same standing: each op is one node to ``torch.compile`` (dynamo traces through it with
``fullgraph=True``; its fake kernel propagates shapes without a GPU) and can be recorded into a HIP graph (no op
allocates or synchronises; workspaces are arguments).

Convention: outputs are written in place into tensors the caller passes (``out``, ``lse``, caches), declared
mutated in the schema, and every op returns nothing -- except the masked-prefill backward, which returns its three
gradients (it runs under autograd, not under graph capture). Device metadata (page tables, lengths, tile lists) are
tensors; the host-side planning that produces them (split choice, tile lists) belongs to the metadata builder.

Every implementation calls the ctypes wrappers of :mod:`abridgekv_amd.ops` (same validation, same C-ABI entry
points), so a compiled or captured call computes bit-identically to a direct call.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional

import torch
from torch import Tensor

from . import ops as _ops
from ._lib import check, lib

_NS = "abridgekv"


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


# -- decode attention ------------------------------------------------------------------------------------------------
@torch.library.custom_op(f"{_NS}::decode_attn", mutates_args=("out", "lse", "workspace"))
def decode_attn(q: Tensor, kv_cache: Tensor, block_table: Tensor, seq_lens: Tensor, scale: float, max_pages: int,
                split_pages: int, out: Tensor, lse: Optional[Tensor], workspace: Optional[Tensor]) -> None:
    """abkv_decode_attn: out [B, 32, 128] (and lse [B, 32]) of one layer's decode over its group's pages. A batch
    that needs more than one split must bring ``workspace`` (ops.decode_workspace): the op never allocates."""
    if -(-max_pages // split_pages) > 1:
        _need(workspace is not None, "decode_attn: the batch needs a workspace (ops.decode_workspace)")
    _ops.decode_attention(q, kv_cache, block_table, seq_lens, scale, max_pages=max_pages, out=out, lse=lse,
                          split_pages=split_pages, workspace=workspace)


@decode_attn.register_fake
def _decode_attn_fake(q, kv_cache, block_table, seq_lens, scale, max_pages, split_pages, out, lse, workspace):
    _need(q.dim() == 3 and tuple(q.shape[1:]) == (_ops.HEADS_Q, _ops.HEAD_DIM), "q must be [B, 32, 128]")
    _need(tuple(out.shape) == tuple(q.shape), "out must be [B, 32, 128]")
    _need(kv_cache.dim() == 5, "kv_cache must be [P, 2, 16, 8, 128]")


# -- KV append, fused RoPE + append, slot mapping ---------------------------------------------------------------------
@torch.library.custom_op(f"{_NS}::kv_append", mutates_args=("kv_cache",))
def kv_append(key: Tensor, value: Tensor, slot_mapping: Tensor, kv_cache: Tensor) -> None:
    """abkv_kv_append (reshape_and_cache): rows of key / value [T, 8, 128] at slot_mapping [T] (< 0 skips)."""
    _ops.kv_append(key, value, slot_mapping, kv_cache)


@kv_append.register_fake
def _kv_append_fake(key, value, slot_mapping, kv_cache):
    _need(key.shape == value.shape and key.shape[0] >= slot_mapping.shape[0], "key / value must cover the slots")


@torch.library.custom_op(f"{_NS}::rope_kv_append", mutates_args=("q", "key", "kv_cache"))
def rope_kv_append(q: Tensor, key: Tensor, value: Tensor, positions: Tensor, cos_sin: Tensor,
                   slot_mapping: Optional[Tensor], kv_cache: Optional[Tensor], block_c: int, codes_k: int,
                   max_position: int, code_span: int = 0) -> None:
    """abkv_rope_kv_append: q and key rotated in place at the RoPE positions of ``positions`` (logical positions of
    the abridged layout when block_c > 0; code rows over offsets [0, code_span), 0 = block_c), rotated key and value
    appended at slot_mapping. ``max_position``: host bound on the positions (checked against the cos/sin table
    without reading the device)."""
    _ops.rope_kv_append(q, key, value, positions, cos_sin, slot_mapping=slot_mapping, kv_cache=kv_cache,
                        block_c=block_c, codes_k=codes_k, max_position=max_position, code_span=code_span)


@rope_kv_append.register_fake
def _rope_kv_append_fake(q, key, value, positions, cos_sin, slot_mapping, kv_cache, block_c, codes_k, max_position,
                         code_span=0):
    _need(q.shape[0] >= positions.shape[0] and key.shape[0] >= positions.shape[0], "q / key must cover the positions")


@torch.library.custom_op(f"{_NS}::slot_mapping", mutates_args=("out",))
def slot_mapping(req_idx: Tensor, positions: Tensor, block_table: Tensor, compacted: Optional[Tensor],
                 out: Tensor) -> None:
    """abkv_slot_mapping: out[t] = table[req][p // 16] * 16 + p % 16, p = positions[t] - compacted[req]."""
    _ops.slot_mapping(req_idx, positions, block_table, out=out, compacted=compacted)


@slot_mapping.register_fake
def _slot_mapping_fake(req_idx, positions, block_table, compacted, out):
    _need(out.shape == positions.shape and req_idx.shape == positions.shape, "one slot per position")


# -- compaction row moves ---------------------------------------------------------------------------------------------
@torch.library.custom_op(f"{_NS}::kv_move_segments", mutates_args=("layer_caches",))
def kv_move_segments(layer_caches: list[Tensor], ops: Tensor, seg_offsets: Tensor) -> None:
    """abkv_kv_move_segments: compaction copy ops [n, 4] applied to every layer cache (<= 16 per call)."""
    _ops.kv_move_segments(layer_caches, ops, seg_offsets)


@kv_move_segments.register_fake
def _kv_move_segments_fake(layer_caches, ops, seg_offsets):
    _need(ops.dim() == 2 and ops.shape[1] == 4, "ops must be [n, 4]")
    _need(0 < len(layer_caches) <= 16, "between 1 and 16 layer caches per call")


@torch.library.custom_op(f"{_NS}::kv_move_mixed", mutates_args=("layer_caches",))
def kv_move_mixed(layer_caches: list[Tensor], ops: Tensor, seg_offsets: Tensor, free_ops: Tensor) -> None:
    """abkv_kv_move_mixed: ordered segments and independent ops of a step's packed fused moves in one launch."""
    _ops.kv_move_mixed(layer_caches, ops, seg_offsets, free_ops)


@kv_move_mixed.register_fake
def _kv_move_mixed_fake(layer_caches, ops, seg_offsets, free_ops):
    _need(ops.dim() == 2 and ops.shape[1] == 4 and free_ops.dim() == 2 and free_ops.shape[1] == 4,
          "ops and free_ops must be [n, 4]")
    _need(0 < len(layer_caches) <= 16, "between 1 and 16 layer caches per call")


def _moves_expand_checks(runs, n_runs, pages, groups, out, n_elems):
    for name, t in (("runs", runs), ("pages", pages), ("groups", groups), ("out", out)):
        _need(t.is_cuda and t.dtype == torch.int32 and t.is_contiguous(), f"{name} must be contiguous cuda int32")
    _need(0 <= n_runs and n_runs * RUN_FIELDS <= runs.numel() and groups.numel() % 4 == 0,
          f"runs must hold n_runs records of {RUN_FIELDS} int32, groups [G, 4]")
    _need(0 <= n_elems <= out.numel(), "out must hold n_elems int32")


RUN_FIELDS = 30                                              # int32 per record of abkv_planner_take_move_runs


@torch.library.custom_op(f"{_NS}::moves_expand", mutates_args=("out",))
def moves_expand(runs: Tensor, n_runs: int, pages: Tensor, groups: Tensor, page_shift: int, out: Tensor,
                 n_elems: int) -> None:
    """abkv_moves_expand: the planner's run descriptors (the n_runs records of take_step_move_runs' layout -- record
    slots past them are stale -- the page windows and the group table [G, 4], all on the device) written out as the
    step's move lists (n_elems int32 of out), ready for kv_move_mixed."""
    _moves_expand_checks(runs, n_runs, pages, groups, out, n_elems)
    stream = C.c_void_p(torch.cuda.current_stream(out.device).cuda_stream)
    check(lib().abkv_moves_expand(C.c_void_p(runs.data_ptr()), int(n_runs), C.c_void_p(pages.data_ptr()),
                                  pages.numel(), C.c_void_p(groups.data_ptr()), groups.numel() // 4, int(page_shift),
                                  C.c_void_p(out.data_ptr()), int(n_elems), stream), "abkv_moves_expand")


@moves_expand.register_fake
def _moves_expand_fake(runs, n_runs, pages, groups, page_shift, out, n_elems):
    _moves_expand_checks(runs, n_runs, pages, groups, out, n_elems)


# -- paged multi-query attention (prompt chunks, code steps) --------------------------------------------------------
@torch.library.custom_op(f"{_NS}::paged_prefill_attn", mutates_args=("out", "lse", "workspace"))
def paged_prefill_attn(q: Tensor, kv_cache: Tensor, block_table: Tensor, q_start: Tensor, kv_start: Tensor,
                       kv_limit: Tensor, tile_req: Tensor, tile_q0: Tensor, causal: Tensor, scale: float,
                       num_tokens: int, num_splits: int, split_tiles: int, out: Tensor, lse: Optional[Tensor],
                       workspace: Optional[Tensor], kv_excluded: Optional[Tensor] = None) -> None:
    """abkv_paged_prefill_attn with device metadata (int32: q_start [B+1], kv_start / kv_limit / causal [B], the
    64-row query tiles tile_req / tile_q0, optional kv_excluded [B, 2] key ranges hidden per request) and a caller
    workspace when num_splits > 1; ``num_tokens`` is q_start[B] (the rows the launch writes)."""
    _need(q.is_cuda and q.dtype == torch.bfloat16 and q.dim() == 3 and q.stride(2) == 1, "q: cuda bf16 [T, 32, 128]")
    _ops._check_cache(kv_cache)
    for name, t in (("block_table", block_table), ("q_start", q_start), ("kv_start", kv_start),
                    ("kv_limit", kv_limit), ("tile_req", tile_req), ("tile_q0", tile_q0), ("causal", causal)):
        _need(t.is_cuda and t.dtype == torch.int32 and t.is_contiguous(), f"{name} must be contiguous cuda int32")
    _need(tile_req.numel() == tile_q0.numel(), "tile_req and tile_q0 must have the same length")
    _need(0 <= num_tokens <= q.shape[0] and tuple(out.shape) == tuple(q.shape) and out.stride(2) == 1,
          "out must be [T, 32, 128] and num_tokens <= T")
    ws_bytes = 0
    if num_splits > 1:
        need = lib().abkv_paged_prefill_workspace_size(num_tokens, num_splits)
        _need(workspace is not None and workspace.numel() * workspace.element_size() >= need,
              "paged_prefill_attn: key splits need a workspace of abkv_paged_prefill_workspace_size bytes")
        ws_bytes = workspace.numel() * workspace.element_size()
    if lse is not None:
        _need(lse.dtype == torch.float32 and lse.is_contiguous() and lse.numel() >= q.shape[0] * _ops.HEADS_Q,
              "lse must be contiguous fp32 [T, 32]")
    if kv_excluded is not None:
        _need(kv_excluded.is_cuda and kv_excluded.dtype == torch.int32 and kv_excluded.is_contiguous()
              and kv_excluded.numel() == 2 * kv_start.numel(), "kv_excluded must be contiguous cuda int32 [B, 2]")
    if tile_req.numel() == 0:
        return
    rc = lib().abkv_paged_prefill_attn(
        _ops._ptr(q), q.stride(0), q.stride(1), _ops._ptr(kv_cache), kv_cache.shape[0], _ops._ptr(block_table),
        _ops._row_stride(block_table), block_table.shape[1], _ops._ptr(q_start), _ops._ptr(kv_start),
        _ops._ptr(kv_limit), _ops._ptr(kv_excluded), _ops._ptr(tile_req), _ops._ptr(tile_q0), tile_req.numel(),
        _ops._ptr(causal), 1,
        float(scale), _ops._ptr(out), out.stride(0), out.stride(1), _ops._ptr(lse), num_tokens, num_splits,
        split_tiles, _ops._ptr(workspace) if num_splits > 1 else None, ws_bytes, C.c_void_p(_ops._stream()))
    check(rc, "abkv_paged_prefill_attn")


@paged_prefill_attn.register_fake
def _paged_prefill_attn_fake(q, kv_cache, block_table, q_start, kv_start, kv_limit, tile_req, tile_q0, causal, scale,
                             num_tokens, num_splits, split_tiles, out, lse, workspace, kv_excluded=None):
    _need(tuple(out.shape) == tuple(q.shape), "out must be [T, 32, 128]")


# -- block-masked teacher-forced attention --------------------------------------------------------------------------
@torch.library.custom_op(f"{_NS}::prefill_masked_attn", mutates_args=("out", "lse"))
def prefill_masked_attn(q: Tensor, k: Tensor, v: Tensor, block_c: int, codes_k: int, num_blocks: int,
                        prompt_len: Optional[Tensor], head_quota: Optional[Tensor], scale: float, out: Tensor,
                        lse: Optional[Tensor], retain_tail: int = 0, tail_policy: int = 0,
                        pause_xattn: int = 0, pause_passes: int = 1, copy_rows: int = 0, replay_rows: int = 0,
                        replay_exclude: bool = False) -> None:
    """abkv_prefill_masked_attn: attention under the compression mask, q [B, S0, 32, 128], k / v [B, S0, 8, 128]
    (retain_tail: T of a retained tail, 0 for none; tail_policy: 0 static, 1 rolling, 2 sticky, 3 raw; pause_xattn:
    0 full, 1 causal, 2 none; pause_passes: L passes of codes_k code rows per block; copy_rows: a copy region after
    the blocks; replay_rows / replay_exclude: the replay tail)."""
    _ops.prefill_masked_attention(q, k, v, block_c, codes_k, num_blocks, prompt_len=prompt_len,
                                  head_quota=head_quota, scale=scale, out=out, lse=lse, retain_tail=retain_tail,
                                  tail_policy=_ops.TAIL_POLICIES[tail_policy], pause_xattn=_ops.XATTN[pause_xattn],
                                  pause_passes=pause_passes, copy_rows=copy_rows, replay_rows=replay_rows,
                                  replay_exclude=replay_exclude)


@prefill_masked_attn.register_fake
def _prefill_masked_attn_fake(q, k, v, block_c, codes_k, num_blocks, prompt_len, head_quota, scale, out, lse,
                              retain_tail=0, tail_policy=0, pause_xattn=0, pause_passes=1, copy_rows=0,
                              replay_rows=0, replay_exclude=False):
    _need(q.shape[1] == num_blocks * (block_c + pause_passes * codes_k + replay_rows) + copy_rows,
          "seq_len must be num_blocks * (block_c + L * codes_k + replay_rows) + copy_rows")
    _need(tuple(out.shape) == tuple(q.shape), "out must be [B, S0, 32, 128]")


@torch.library.custom_op(f"{_NS}::prefill_masked_attn_bwd", mutates_args=())
def prefill_masked_attn_bwd(q: Tensor, k: Tensor, v: Tensor, out: Tensor, lse: Tensor, dout: Tensor, block_c: int,
                            codes_k: int, num_blocks: int, prompt_len: Optional[Tensor],
                            head_quota: Optional[Tensor], scale: float,
                            retain_tail: int = 0, tail_policy: int = 0,
                            pause_xattn: int = 0, pause_passes: int = 1, copy_rows: int = 0, replay_rows: int = 0,
                            replay_exclude: bool = False) -> tuple[Tensor, Tensor, Tensor]:
    """abkv_prefill_masked_attn_bwd: (dq, dk, dv) of sum(dout * out) under the same mask (new tensors)."""
    return _ops.prefill_masked_attention_backward(q, k, v, out, lse, dout, block_c, codes_k, num_blocks,
                                                  prompt_len=prompt_len, head_quota=head_quota, scale=scale,
                                                  retain_tail=retain_tail,
                                                  tail_policy=_ops.TAIL_POLICIES[tail_policy],
                                                  pause_xattn=_ops.XATTN[pause_xattn], pause_passes=pause_passes,
                                                  copy_rows=copy_rows, replay_rows=replay_rows,
                                                  replay_exclude=replay_exclude)


@prefill_masked_attn_bwd.register_fake
def _prefill_masked_attn_bwd_fake(q, k, v, out, lse, dout, block_c, codes_k, num_blocks, prompt_len, head_quota,
                                  scale, retain_tail=0, tail_policy=0, pause_xattn=0, pause_passes=1, copy_rows=0,
                                  replay_rows=0, replay_exclude=False):
    _need(q.shape[1] == num_blocks * (block_c + pause_passes * codes_k + replay_rows) + copy_rows,
          "seq_len must be num_blocks * (block_c + L * codes_k + replay_rows) + copy_rows")
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


OPS = ("decode_attn", "kv_append", "rope_kv_append", "slot_mapping", "kv_move_segments", "kv_move_mixed",
       "moves_expand", "paged_prefill_attn", "prefill_masked_attn", "prefill_masked_attn_bwd")
