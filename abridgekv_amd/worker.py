"""Worker-side execution of compaction: copy ops, fused moves, block-table truncation, slot maps.

Mirrors GPUModelRunner._execute_kv_copy_operations / _execute_kv_copy_group
(third_party/vllm_overlay/vllm/v1/worker/gpu_model_runner.py:1147-1224), the truncation step of _update_states
(:935-950, block_table.py:132-137, :330-336) and the per-group slot maps (:1579-1661, block_table.py:186-197),
executing on the HIP kernels of libabridgekv_amd.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import ops
from ._lib import lib
from .ops import PAGE


def _validate_ops(all_ops: np.ndarray, num_pages: int) -> None:
    if all_ops.size == 0:
        return
    if (all_ops[:, [0, 2]].min() < 0 or all_ops[:, [0, 2]].max() >= num_pages
            or all_ops[:, [1, 3]].min() < 0 or all_ops[:, [1, 3]].max() >= PAGE):
        raise ValueError("copy op names a page or offset outside the cache")


def _reads_after_write(seg: np.ndarray) -> bool:
    """True if some op of the segment reads a slot an earlier op of the segment wrote."""
    dst = seg[:, 2].astype(np.int64) * PAGE + seg[:, 3]
    src = seg[:, 0].astype(np.int64) * PAGE + seg[:, 1]
    first_write = {}
    for i, d in enumerate(dst.tolist()):
        first_write.setdefault(d, i)
    return any(first_write.get(s, len(dst)) < i for i, s in enumerate(src.tolist()))


def execute_kv_copy_group(segments, layer_caches, check: bool = True) -> None:
    """Apply one batch: ``segments`` is a list of per-request op lists [(src_block, src_off, dst_block, dst_off)];
    every layer cache of the group receives the same moves with gather-then-scatter semantics."""
    segs = [np.asarray(s, dtype=np.int32).reshape(-1, 4) for s in segments if len(s)]
    if not segs:
        return
    all_ops = np.concatenate(segs)
    device = layer_caches[0].device
    num_pages = layer_caches[0].shape[0]
    if check:
        _validate_ops(all_ops, num_pages)
    hazard = check and any(_reads_after_write(s) for s in segs)
    ops_d = torch.from_numpy(all_ops).to(device, non_blocking=False)
    for lo in range(0, len(layer_caches), 16):
        caches = layer_caches[lo: lo + 16]
        if hazard:
            ops.kv_copy_staged(caches, ops_d)
        else:
            offs = np.zeros(len(segs) + 1, np.int32)
            offs[1:] = np.cumsum([len(s) for s in segs])
            ops.kv_move_segments(caches, ops_d, torch.from_numpy(offs).to(device))


def execute_kv_copy_operations(kv_copy_operations: dict, layer_caches_by_group, check: bool = True) -> None:
    """Per group, batch b of every request is applied together, batches in order (a later removal's ops assume the
    earlier shift is done). ``kv_copy_operations``: request id -> per group -> ordered batches of ops."""
    for gid, caches in enumerate(layer_caches_by_group):
        batches = [per_group[gid] for per_group in kv_copy_operations.values() if gid < len(per_group)]
        num_batches = max((len(b) for b in batches), default=0)
        for b in range(num_batches):
            segments = [req[b] for req in batches if b < len(req)]
            execute_kv_copy_group(segments, caches, check=check)


def pack_fused_moves(fused_moves: np.ndarray, num_pages: int, check: bool = True, num_groups: int | None = None):
    """Host side of :func:`execute_fused_moves` (abkv_moves_pack): a planner step's fused move rows (request, group,
    src_block, src_off, dst_block, dst_off) as per-group device-ready lists -- the runs in which some op's
    destination is another op's source as ordered segments (op order kept), every other op as an independent op.
    Returns (buffer int32, [(group, ops_at, n_ops, offs_at, n_segments, n_free)]) for the groups with ops; ops and
    offsets are slices of the one buffer."""
    if fused_moves.size == 0:
        return np.zeros(0, np.int32), []
    fm = np.ascontiguousarray(fused_moves, dtype=np.int64)
    if check:
        _validate_ops(fm[:, 2:6], num_pages)
    G = int(fm[:, 1].max()) + 1 if num_groups is None else num_groups
    n = fm.shape[0]
    out = np.empty(5 * n + 4 * G, np.int32)
    index = np.zeros((G, 5), np.int64)
    got = lib().abkv_moves_pack(fm.ctypes.data_as(C.POINTER(C.c_int64)), n, G,
                                out.ctypes.data_as(C.POINTER(C.c_int32)), out.size,
                                index.ctypes.data_as(C.POINTER(C.c_int64)))
    if got < 0:
        raise ValueError(f"abkv_moves_pack rejected the fused moves ({got}): rows of one (request, group) must be "
                         "contiguous, and no op may read a slot an earlier op of its run writes")
    return out[:got], [(g, *map(int, index[g])) for g in range(G) if index[g, 1] > 0]


def prepare_fused_moves(fused_moves: np.ndarray, num_pages: int, device, check: bool = True):
    """:func:`pack_fused_moves` uploaded in a single host-to-device copy.
    Returns [(group, ordered ops [n, 4] int32, seg_offsets [n_seg + 1] int32, independent ops [m, 4] int32)] on the
    device."""
    buf, parts = pack_fused_moves(fused_moves, num_pages, check)
    if not parts:
        return []
    return device_move_lists(torch.from_numpy(buf).to(device), parts)


class MoveUploader:
    """A planner step's move lists (KVPlanner.take_step_moves) written into pinned host memory and uploaded with one
    asynchronous copy. The pinned buffer is reused: a call first waits for the copy that last read it."""

    def __init__(self, device, capacity: int = 1 << 16):
        self.device = device
        self._pinned = torch.empty(capacity, dtype=torch.int32, pin_memory=True)
        self._dev = torch.empty(capacity, dtype=torch.int32, device=device)
        self._done = None

    def take(self, planner):
        """(trunc_rows, [(group, ordered ops, seg_offsets, independent ops)] on the device) of the pending step."""
        need = planner.moves_capacity()
        if self._done is not None:
            self._done.synchronize()
        if need > self._pinned.numel():
            self._pinned = torch.empty(2 * need, dtype=torch.int32, pin_memory=True)
            self._dev = torch.empty(2 * need, dtype=torch.int32, device=self.device)
        trunc, buf, parts = planner.take_step_moves(self._pinned.numpy())
        if not parts:
            return trunc, []
        n = buf.size
        self._dev[:n].copy_(self._pinned[:n], non_blocking=True)
        self._done = torch.cuda.Event()
        self._done.record()
        return trunc, device_move_lists(self._dev[:n], parts)


def take_step_move_lists(planner):
    """The pending step's fused moves, ready for upload: ("runs", buffer, layout, parts, n_elems) with the run
    descriptors the device expands (KVPlanner.take_step_move_runs), or -- when the planner refuses descriptors for
    the step (more than 8 span removals of one request and group in one step; the step then stays pending) --
    ("packed", buffer, None, parts, n_elems) with the move lists written on the host (KVPlanner.take_step_moves).
    ``parts`` as pack_fused_moves; n_elems = int32 elements of the move lists."""
    try:
        _, desc, layout, parts, n_elems = planner.take_step_move_runs()
        return "runs", desc, layout, parts, n_elems
    except RuntimeError as e:
        if "more than 8 span removals" not in str(e):
            raise
    _, buf, parts = planner.take_step_moves()
    return "packed", buf, None, parts, int(buf.size)


class MoveRunUploader:
    """A planner step's fused moves as run descriptors (KVPlanner.take_step_move_runs): the records, page windows and
    group table go to the device in one asynchronous copy from pinned memory, and abkv_moves_expand writes the move
    lists there -- the same lists as :class:`MoveUploader`, element for element, with the per-row work on the device.
    The pinned and device buffers are reused; a call first waits for the copy that last read the pinned one, and the
    move lists of a call stay valid until the next call's expansion (on the same stream) overwrites them."""

    def __init__(self, device, capacity: int = 1 << 16, out_capacity: int = 1 << 20):
        self.device = device
        self._pinned = torch.empty(capacity, dtype=torch.int32, pin_memory=True)
        self._dev = torch.empty(capacity, dtype=torch.int32, device=device)
        self._out = torch.empty(out_capacity, dtype=torch.int32, device=device)
        self._done = None

    def take(self, planner):
        """(trunc_rows, [(group, ordered ops, seg_offsets, independent ops)] on the device) of the pending step."""
        need = planner.move_runs_capacity()
        if self._done is not None:
            self._done.synchronize()
        if need > self._pinned.numel():
            self._pinned = torch.empty(2 * need, dtype=torch.int32, pin_memory=True)
            self._dev = torch.empty(2 * need, dtype=torch.int32, device=self.device)
        trunc, desc, (runs_at, n_runs, pages_at, groups_at), parts, n_elems = \
            planner.take_step_move_runs(self._pinned.numpy())
        if not parts:
            return trunc, []
        n = desc.size
        self._dev[:n].copy_(self._pinned[:n], non_blocking=True)
        self._done = torch.cuda.Event()
        self._done.record()
        if n_elems > self._out.numel():
            self._out = torch.empty(2 * n_elems, dtype=torch.int32, device=self.device)
        base = self._dev.data_ptr()
        shift = int(planner.block_size).bit_length() - 1
        rc = lib().abkv_moves_expand(C.c_void_p(base + 4 * runs_at), n_runs, C.c_void_p(base + 4 * pages_at),
                                     groups_at - pages_at, C.c_void_p(base + 4 * groups_at), planner.num_groups, shift,
                                     C.c_void_p(self._out.data_ptr()), n_elems,
                                     C.c_void_p(torch.cuda.current_stream(self.device).cuda_stream))
        if rc != 0:
            raise RuntimeError(f"abkv_moves_expand failed ({rc})")
        return trunc, device_move_lists(self._out[:n_elems], parts)


def device_move_lists(dev_buf: torch.Tensor, parts):
    """Views of an uploaded :func:`pack_fused_moves` buffer: [(group, ordered ops, seg_offsets, independent ops)]."""
    out = []
    for gid, o, n, so, ns, nf in parts:
        n_ord = n - nf
        out.append((gid, dev_buf[o: o + 4 * n_ord].view(-1, 4), dev_buf[so: so + ns + 1],
                    dev_buf[o + 4 * n_ord: o + 4 * n].view(-1, 4)))
    return out


def launch_moves(prepared, layer_caches_by_group, events=None) -> None:
    """Device side of :func:`execute_fused_moves`: one launch per group (and per 16 layer tensors). ``events``, if
    given, is a list that receives (start, end) CUDA events recorded around every launch."""
    for gid, ops_d, offs_d, free_d in prepared:
        caches = layer_caches_by_group[gid]
        for lo in range(0, len(caches), 16):
            if events is not None:
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
            ops.kv_move_mixed(caches[lo: lo + 16], ops_d, offs_d, free_d)
            if events is not None:
                e.record()
                events.append((s, e))


def execute_fused_moves(fused_moves: np.ndarray, layer_caches_by_group, check: bool = True) -> None:
    """Apply a planner step's fused move rows (request, group, src_block, src_off, dst_block, dst_off): one launch
    per group. Rows of one (request, group) are monotone (increasing source, dst < src): a run whose ops depend on
    each other's order is walked in order by the in-register chunked copy, every other op moves independently."""
    if fused_moves.size == 0:
        return
    num_pages = layer_caches_by_group[0][0].shape[0]
    launch_moves(prepare_fused_moves(fused_moves, num_pages, layer_caches_by_group[0][0].device, check),
                 layer_caches_by_group)


def truncate_block_table(block_ids_by_group, keep):
    """block_table.py:132-137 / gpu_model_runner.py:935-950: keep the first ``keep[g]`` pages of every group."""
    if len(block_ids_by_group) != len(keep):
        raise RuntimeError("KV cache group count changed during block-table compaction")
    for ids, k in zip(block_ids_by_group, keep):
        del ids[k:]


def physical_positions(logical_positions, compacted_counts):
    """gpu_model_runner.py:1585-1590: one physical position array per group, phys = logical - compacted[g]."""
    lp = np.asarray(logical_positions, dtype=np.int64)
    return [lp - c for c in compacted_counts]


def slot_mapping_host(block_ids, positions):
    """block_table.py:186-197 on the host (used when the metadata is built on the CPU)."""
    pos = np.asarray(positions, dtype=np.int64)
    table = np.asarray(block_ids, dtype=np.int64)
    return table[pos // PAGE] * PAGE + pos % PAGE
