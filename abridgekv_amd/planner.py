"""Compaction planner: the scheduler / KV-cache-manager side of block-boundary compaction.

Python face of the native planner (``abkv_planner_*`` in include/abridgekv_amd.h), keeping the call shapes of the
reference's vLLM overlay:
* ``KVPlanner.allocate_slots(request_id, num_new_tokens)`` -- KVCacheManager.allocate_slots
  (third_party/vllm_overlay/vllm/v1/core/kv_cache_manager.py:206-340): per-group pages net of compacted tokens,
  ``None`` when the pool cannot cover the request.
* ``KVPlanner.mask_token_span(request_id, start, end, groups=None) -> SpanRemovalResult`` -- Scheduler.mask_token_span
  (third_party/vllm_overlay/vllm/v1/core/sched/scheduler.py:2060-2204), the ``MaskSpan`` callback the CompressLM
  processor calls (third_party/vllm_overlay/vllm/v1/core/compresslm/processor.py:18, :648-661).
* ``KVPlanner.take_step_outputs()`` -- the SchedulerOutput fields ``kv_copy_operations`` and
  ``block_table_truncations`` (third_party/vllm_overlay/vllm/v1/core/sched/output.py:221-225), plus the fused move
  list the device executor runs.
* per-group span maps as on ``Request`` (third_party/vllm_overlay/vllm/v1/request.py:263-321).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from ._lib import lib

ABKV_OK, ABKV_ERR_SPAN = 0, -3


@dataclass
class SpanRemovalResult:
    """vllm/v1/engine/__init__.py:203-213."""
    success: bool
    tokens_removed: int
    blocks_freed: int
    error_message: str | None = None


@dataclass
class StepOutputs:
    """Compaction outputs of one scheduler step.

    ``kv_copy_operations``: request id -> per group -> ordered batches of (src_block, src_off, dst_block, dst_off)
    (the reference's format). ``block_table_truncations``: request id -> pages kept per group.
    ``fused_moves``: int64 [n, 6] (request handle, group, src_block, src_off, dst_block, dst_off), every removal of the
    step composed per (request, group), rows truncated later in the same step left out.
    """
    kv_copy_operations: dict = field(default_factory=dict)
    block_table_truncations: dict = field(default_factory=dict)
    fused_moves: np.ndarray = field(default_factory=lambda: np.zeros((0, 6), np.int64))


def _i32(arr):
    return arr.ctypes.data_as(C.POINTER(C.c_int32))


def _i64(arr):
    return arr.ctypes.data_as(C.POINTER(C.c_int64))


class KVPlanner:
    """One page pool shared by ``num_groups`` KV-cache groups (pages of ``block_size`` slots, page 0 = null)."""

    def __init__(self, num_blocks: int, num_groups: int, block_size: int = 16, free_order=None,
                 max_model_len: int | None = None, op_rows: bool = True):
        """``op_rows=False``: skip the reference-format op batches (the bookkeeping and the fused moves are unchanged;
        the step outputs then hold no ``kv_copy_operations``), for callers that execute the fused moves only."""
        self._lib = lib()
        fo = None
        if free_order is not None:
            self._free_order = np.ascontiguousarray(free_order, dtype=np.int32)
            if self._free_order.size != num_blocks - 1:
                raise ValueError("free_order must list every page 1..num_blocks-1")
            fo = _i32(self._free_order)
        self._h = self._lib.abkv_planner_create(num_blocks, num_groups, block_size, fo, int(max_model_len or 0))
        if not self._h:
            raise ValueError("invalid planner configuration (free_order must be a permutation of 1..num_blocks-1)")
        self.num_blocks, self.num_groups, self.block_size = num_blocks, num_groups, block_size
        self.op_rows = bool(op_rows)
        if not self.op_rows and self._lib.abkv_planner_set_op_rows(self._h, 0) != ABKV_OK:
            raise RuntimeError("abkv_planner_set_op_rows failed")
        self._ids: dict = {}
        self._names: dict = {}
        self._bufs: dict = {}

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.abkv_planner_destroy(h)
            self._h = None

    # -- request handles ---------------------------------------------------------------------------------------
    def handle(self, request_id) -> int:
        if isinstance(request_id, (int, np.integer)) and request_id not in self._ids:
            return int(request_id)
        return self._ids[request_id]

    def request_id(self, handle: int):
        return self._names.get(handle, handle)

    def _err(self) -> str:
        return self._lib.abkv_planner_last_error(self._h).decode()

    def add_request(self, request_id) -> None:
        h = int(request_id) if isinstance(request_id, (int, np.integer)) else len(self._ids) + (1 << 40)
        self._ids[request_id] = h
        self._names[h] = request_id
        if self._lib.abkv_planner_add_request(self._h, h) != ABKV_OK:
            raise RuntimeError(self._err())

    def free(self, request_id) -> None:
        h = self.handle(request_id)
        if self._lib.abkv_planner_free_request(self._h, h) != ABKV_OK:
            raise KeyError(request_id)
        self._ids.pop(request_id, None)
        self._names.pop(h, None)

    def num_computed_tokens(self, request_id) -> int:
        return int(self._lib.abkv_planner_get_num_computed(self._h, self.handle(request_id)))

    def set_num_computed_tokens(self, request_id, n: int) -> None:
        if self._lib.abkv_planner_set_num_computed(self._h, self.handle(request_id), int(n)) != ABKV_OK:
            raise KeyError(request_id)

    # -- KVCacheManager ----------------------------------------------------------------------------------------
    def allocate_slots(self, request_id, num_new_tokens: int):
        """New pages per group, or None when the pool cannot cover the request (nothing is allocated then)."""
        if num_new_tokens == 0:
            raise ValueError("num_new_tokens must be greater than 0")
        before = [len(b) for b in self.get_blocks(request_id)]
        rc = self._lib.abkv_planner_allocate_slots(self._h, self.handle(request_id), int(num_new_tokens))
        if rc == 0:
            return None
        if rc < 0:
            raise ValueError(self._err())
        return tuple(b[n:] for b, n in zip(self.get_blocks(request_id), before))

    def get_blocks(self, request_id) -> tuple[list[int], ...]:
        h = self.handle(request_id)
        out = []
        for g in range(self.num_groups):
            buf = np.empty(self.num_blocks, np.int32)
            n = self._lib.abkv_planner_block_ids(self._h, h, g, _i32(buf), buf.size)
            if n < 0:
                raise KeyError(request_id)
            out.append(buf[:n].tolist())
        return tuple(out)

    def num_free_blocks(self) -> int:
        return int(self._lib.abkv_planner_num_free(self._h))

    def free_queue(self) -> list[int]:
        buf = np.empty(self.num_blocks, np.int32)
        n = self._lib.abkv_planner_free_queue(self._h, _i32(buf), buf.size)
        return buf[:n].tolist()

    def fill_block_table(self, request_ids, group: int, width: int, pad: int = 0) -> np.ndarray:
        rids = np.ascontiguousarray([self.handle(r) for r in request_ids], dtype=np.int64)
        table = np.empty((len(rids), width), np.int32)
        rc = self._lib.abkv_planner_fill_block_table(self._h, _i64(rids), len(rids), group, _i32(table), width, pad)
        if rc != ABKV_OK:
            raise ValueError(f"fill_block_table failed ({rc}): width too small or unknown request")
        return table

    # -- Request span maps (per group) ---------------------------------------------------------------------------
    def compacted_counts(self, request_id) -> tuple[int, ...]:
        h = self.handle(request_id)
        return tuple(int(self._lib.abkv_planner_compacted(self._h, h, g)) for g in range(self.num_groups))

    def group_compacted_spans(self, request_id, group: int = 0) -> list[tuple[int, int]]:
        buf = np.empty(2 * 4096, np.int64)
        n = self._lib.abkv_planner_spans(self._h, self.handle(request_id), group, _i64(buf), 4096)
        if n < 0:
            raise ValueError(f"spans failed ({n})")
        return [(int(buf[2 * i]), int(buf[2 * i + 1])) for i in range(n)]

    def logical_to_physical(self, request_id, pos: int, group: int = 0) -> int:
        return int(self._lib.abkv_planner_logical_to_physical(self._h, self.handle(request_id), group, int(pos)))

    def physical_to_logical(self, request_id, pos: int, group: int = 0) -> int:
        return int(self._lib.abkv_planner_physical_to_logical(self._h, self.handle(request_id), group, int(pos)))

    def is_token_active(self, request_id, pos: int, group: int = 0) -> bool:
        return bool(self._lib.abkv_planner_is_token_active(self._h, self.handle(request_id), group, int(pos)))

    # -- Scheduler.mask_token_span -------------------------------------------------------------------------------
    def mask_token_span(self, request_id, start: int, end: int, groups=None) -> SpanRemovalResult:
        try:
            h = self.handle(request_id)
        except KeyError:
            return SpanRemovalResult(False, 0, 0, f"Request {request_id} not found")
        removed, freed = C.c_int64(0), C.c_int64(0)
        if groups is None:
            rc = self._lib.abkv_planner_mask_token_span(self._h, h, int(start), int(end), None, -1,
                                                        C.byref(removed), C.byref(freed))
        else:
            garr = np.ascontiguousarray(list(groups), dtype=np.int32)
            rc = self._lib.abkv_planner_mask_token_span(self._h, h, int(start), int(end), _i32(garr), garr.size,
                                                        C.byref(removed), C.byref(freed))
        if rc == ABKV_OK:
            return SpanRemovalResult(True, removed.value, freed.value)
        if rc == ABKV_ERR_SPAN:
            return SpanRemovalResult(False, 0, 0, self._err())
        raise RuntimeError(f"mask_token_span failed ({rc}): {self._err()}")

    def _buffer(self, name: str, rows: int, cols: int) -> np.ndarray:
        """Reusable, already-faulted output buffer (grown geometrically) so a step does not pay first-touch costs."""
        buf = self._bufs.get(name)
        if buf is None or buf.shape[0] < rows or buf.shape[1] != cols:
            buf = np.zeros((max(rows, 1, 2 * (0 if buf is None else buf.shape[0])), cols), np.int64)
            self._bufs[name] = buf
        return buf

    def reserve_outputs(self, n_ops: int, n_fused: int, n_trunc: int = 1024) -> None:
        """Pre-size (and fault in) the step-output buffers, e.g. before a timed step."""
        self._buffer("ops", n_ops, 7).fill(0)
        self._buffer("fused", n_fused, 6).fill(0)
        self._buffer("trunc", n_trunc, 1 + self.num_groups).fill(0)

    def take_step_outputs(self, as_arrays: bool = False):
        """The step's compaction outputs, then cleared. ``as_arrays=True`` returns the raw int64 rows
        (op_rows [n, 7], trunc_rows [n, 1 + G], fused_moves [n, 6]) as views of reusable buffers, valid until the next
        call, without building the dict form."""
        n_ops, n_tr, n_fu = C.c_int64(0), C.c_int64(0), C.c_int64(0)
        self._lib.abkv_planner_pending_sizes(self._h, C.byref(n_ops), C.byref(n_tr), C.byref(n_fu))
        G = self.num_groups
        ops = self._buffer("ops", n_ops.value, 7)
        tr = self._buffer("trunc", n_tr.value, 1 + G)
        fu = self._buffer("fused", n_fu.value, 6)
        o1, o2, o3 = C.c_int64(0), C.c_int64(0), C.c_int64(0)
        rc = self._lib.abkv_planner_take_step_outputs(self._h, _i64(ops) if self.op_rows else None, ops.shape[0],
                                                      C.byref(o1), _i64(tr), tr.shape[0], C.byref(o2), _i64(fu),
                                                      fu.shape[0], C.byref(o3))
        if rc != ABKV_OK:
            raise RuntimeError(f"take_step_outputs failed ({rc}): {self._err()}")
        ops, tr, fu = (ops[:o1.value] if self.op_rows else ops[:0]), tr[:o2.value], fu[:o3.value]
        if as_arrays:
            return ops, tr, fu
        ops, tr, fu = ops.copy(), tr.copy(), fu.copy()
        kv_ops: dict = {}
        for row in ops:
            rid = self.request_id(int(row[0]))
            per_group = kv_ops.setdefault(rid, [[] for _ in range(G)])
            batches = per_group[int(row[1])]
            while len(batches) <= int(row[2]):
                batches.append([])
            batches[int(row[2])].append(tuple(int(x) for x in row[3:]))
        trunc = {self.request_id(int(row[0])): tuple(int(x) for x in row[1:]) for row in tr}
        return StepOutputs(kv_ops, trunc, fu)

    def moves_capacity(self) -> int:
        """int32 elements :meth:`take_step_moves` needs for the pending step."""
        n_ops, n_tr, n_fu = C.c_int64(0), C.c_int64(0), C.c_int64(0)
        self._lib.abkv_planner_pending_sizes(self._h, C.byref(n_ops), C.byref(n_tr), C.byref(n_fu))
        return 5 * n_fu.value + 4 * self.num_groups

    def take_step_moves(self, out: np.ndarray | None = None):
        """The step's outputs for a caller that executes fused moves (abkv_planner_take_moves_packed), then cleared:
        (trunc_rows [n, 1 + G] int64, buffer int32, parts) -- buffer and parts as :func:`worker.pack_fused_moves`
        (per group the ordered segments, then the independent ops, then the segment offsets; parts lists (group,
        ops_at, n_ops, offs_at, n_segments, n_free) for the groups with ops). ``out``: a contiguous int32 array of at
        least :meth:`moves_capacity` elements to write into (e.g. pinned host memory); a reusable one otherwise. The
        views are valid until the next call."""
        n_ops, n_tr, n_fu = C.c_int64(0), C.c_int64(0), C.c_int64(0)
        self._lib.abkv_planner_pending_sizes(self._h, C.byref(n_ops), C.byref(n_tr), C.byref(n_fu))
        G = self.num_groups
        need = 5 * n_fu.value + 4 * G
        if out is None:
            buf = self._bufs.get("moves")
            if buf is None or buf.size < need:
                buf = np.zeros(max(need, 2 * (0 if buf is None else buf.size)), np.int32)
                self._bufs["moves"] = buf
            out = buf
        if out.dtype != np.int32 or not out.flags.c_contiguous or out.size < need:
            raise ValueError(f"out must be a contiguous int32 array of at least {need} elements")
        tr = self._buffer("trunc", n_tr.value, 1 + G)
        index = np.zeros((G, 5), np.int64)
        got_tr = C.c_int64(0)
        rc = self._lib.abkv_planner_take_moves_packed(self._h, _i64(tr), tr.shape[0], C.byref(got_tr), _i32(out),
                                                      out.size, _i64(index))
        if rc < 0:
            raise RuntimeError(f"take_moves_packed failed ({rc}): {self._err()}")
        parts = [(g, *map(int, index[g])) for g in range(G) if index[g, 1] > 0]
        return tr[:got_tr.value], out[:rc], parts

    RUN_FIELDS = 30                                        # int32 per record of abkv_planner_take_move_runs

    def move_runs_capacity(self) -> int:
        """int32 elements :meth:`take_step_move_runs` needs for the pending step (records, page windows, group table
        and section alignment)."""
        n_runs, n_pages = C.c_int64(0), C.c_int64(0)
        self._lib.abkv_planner_pending_run_sizes(self._h, C.byref(n_runs), C.byref(n_pages))
        return self.RUN_FIELDS * n_runs.value + n_pages.value + 4 * self.num_groups + 12

    def take_step_move_runs(self, out: np.ndarray | None = None):
        """The step's fused moves as run descriptors (abkv_planner_take_move_runs), then cleared: (trunc_rows,
        buffer int32, layout, parts, n_elems). ``buffer`` holds three 16-byte aligned sections -- the records
        [n_runs, RUN_FIELDS], the page windows, the group table [num_groups, 4] -- at ``layout`` = (runs_at, n_runs,
        pages_at, groups_at); ``parts`` as :meth:`take_step_moves`; ``n_elems`` = int32 elements of the move lists
        abkv_moves_expand writes from them (the buffer :meth:`take_step_moves` would return, element for element).
        ``out``: a contiguous int32 array of at least :meth:`move_runs_capacity` elements (e.g. pinned memory)."""
        n_runs, n_pages = C.c_int64(0), C.c_int64(0)
        self._lib.abkv_planner_pending_run_sizes(self._h, C.byref(n_runs), C.byref(n_pages))
        G = self.num_groups
        r_cap, p_cap = n_runs.value, n_pages.value
        runs_at = 0
        pages_at = (runs_at + self.RUN_FIELDS * r_cap + 3) & ~3
        groups_at = (pages_at + p_cap + 3) & ~3
        need = groups_at + 4 * G
        if out is None:
            buf = self._bufs.get("runs")
            if buf is None or buf.size < need:
                buf = np.zeros(max(need, 2 * (0 if buf is None else buf.size)), np.int32)
                self._bufs["runs"] = buf
            out = buf
        if out.dtype != np.int32 or not out.flags.c_contiguous or out.size < need:
            raise ValueError(f"out must be a contiguous int32 array of at least {need} elements")
        n_ops, n_tr, n_fu = C.c_int64(0), C.c_int64(0), C.c_int64(0)
        self._lib.abkv_planner_pending_sizes(self._h, C.byref(n_ops), C.byref(n_tr), C.byref(n_fu))
        tr = self._buffer("trunc", n_tr.value, 1 + G)
        index = np.zeros((G, 5), np.int64)
        sizes = np.zeros(3, np.int64)
        got_tr = C.c_int64(0)
        base = out.ctypes.data
        rc = self._lib.abkv_planner_take_move_runs(
            self._h, _i64(tr), tr.shape[0], C.byref(got_tr), C.cast(base + 4 * runs_at, C.POINTER(C.c_int32)), r_cap,
            C.cast(base + 4 * pages_at, C.POINTER(C.c_int32)), p_cap, C.cast(base + 4 * groups_at, C.POINTER(C.c_int32)),
            _i64(index), _i64(sizes))
        if rc != ABKV_OK:
            raise RuntimeError(f"take_move_runs failed ({rc}): {self._err()}")
        parts = [(g, *map(int, index[g])) for g in range(G) if index[g, 1] > 0]
        layout = (runs_at, int(sizes[0]), pages_at, groups_at)
        return tr[:got_tr.value], out[:need], layout, parts, int(sizes[2])

    def apply_events(self, events: np.ndarray) -> None:
        """Apply a batch of scheduler events (see abkv_planner_apply_events); raises on the first failure."""
        ev = np.ascontiguousarray(events, dtype=np.int64).reshape(-1, 6)
        n = self._lib.abkv_planner_apply_events(self._h, _i64(ev), ev.shape[0])
        if n < 0:
            raise RuntimeError(f"event {-n - 1} ({ev[-n - 1].tolist()}) failed: {self._err()}")
