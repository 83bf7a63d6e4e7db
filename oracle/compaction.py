"""Serving-side compaction planner and copy execution (oracle; test infrastructure only).

A line-by-line restatement, in plain Python, of the integer bookkeeping the reference's vLLM overlay runs when a
span of tokens is compacted out of a request's paged KV cache, plus the worker's execution of the resulting copy
ops. Prefix caching, eviction, hybrid attention, KV events and speculative lookahead are out of scope (CompressLM
requires prefix caching off: third_party/vllm_overlay/vllm/v1/core/sched/scheduler.py:111-112).

Pinning (tests/test_oracle_compaction.py):
* ``CompactedSpanIndex``   -- brute force over 300 random layouts (the reference's own check,
                              scripts/test_compresslm_physical_quotas.py:28-49).
* ``FreeBlockQueue`` / ``BlockPool`` -- conservation (free + live = pool - 1 null page), FIFO order, reverse-order
                              frees, null page never handed out.
* ``Planner.mask_token_span`` and the worker copy -- after every compaction each group's physical stream equals the
                              brute-force filter of the logical stream (every kept row's bytes equal its
                              pre-compaction bytes), page lists hold exactly ceil(active/16) pages, the span maps agree
                              with brute force, and the reference's own invariant: each compacted block keeps exactly
                              codes[:q_g] and no response content (scripts/test_compresslm_physical_quotas.py:115-138).
* validation errors        -- each SpanRemovalResult error branch of scheduler.py:2090-2161 is forced from the host.
"""
from __future__ import annotations

import bisect
from collections import deque
from dataclasses import dataclass

import numpy as np

from .layout import PAGE


# ----------------------------------------------------------------------------------------------------------------
# third_party/vllm_overlay/vllm/v1/compacted_spans.py:8-68
# ----------------------------------------------------------------------------------------------------------------
class CompactedSpanIndex:
    """Sorted, non-overlapping removed logical spans of one KV-cache group with logical<->physical maps."""

    def __init__(self, spans):
        self.spans = list(spans)
        self._starts, self._cumulative = [], []
        self._gap_physical, self._gap_logical = [0], [0]
        total = 0
        for s, e in self.spans:
            self._starts.append(s)
            total += e - s
            self._cumulative.append(total)
            self._gap_physical.append(e - total)
            self._gap_logical.append(e)
        self.total_removed = total

    def is_token_active(self, position):                          # compacted_spans.py:32-38
        if not self._starts:
            return True
        idx = bisect.bisect_right(self._starts, position) - 1
        if idx < 0:
            return True
        return position >= self.spans[idx][1]

    def get_active_positions(self, num_tokens):                   # compacted_spans.py:40-52
        if not self.spans:
            return list(range(num_tokens))
        active, prev_end = [], 0
        for start, end in self.spans:
            if start >= num_tokens:
                break
            active.extend(range(prev_end, min(start, num_tokens)))
            prev_end = end
        if prev_end < num_tokens:
            active.extend(range(prev_end, num_tokens))
        return active

    def logical_to_physical(self, logical_pos):                   # compacted_spans.py:54-64
        if not self._starts:
            return logical_pos
        idx = bisect.bisect_right(self._starts, logical_pos) - 1
        if idx < 0:
            return logical_pos
        _, end = self.spans[idx]
        if logical_pos >= end:
            return logical_pos - self._cumulative[idx]
        prev_cum = self._cumulative[idx - 1] if idx > 0 else 0
        return logical_pos - prev_cum - (logical_pos - self._starts[idx])

    def physical_to_logical(self, physical_pos):                  # compacted_spans.py:66-68
        idx = bisect.bisect_right(self._gap_physical, physical_pos) - 1
        return self._gap_logical[idx] + (physical_pos - self._gap_physical[idx])


def merge_spans(spans):
    """Merge overlapping or adjacent spans: scheduler.py:2043-2058 (_merge_spans)."""
    if not spans:
        return []
    ordered = sorted(spans)
    merged = [ordered[0]]
    for start, end in ordered[1:]:
        ps, pe = merged[-1]
        if start <= pe:
            merged[-1] = (ps, max(pe, end))
        else:
            merged.append((start, end))
    return merged


# ----------------------------------------------------------------------------------------------------------------
# third_party/vllm_overlay/vllm/v1/core/kv_cache_utils.py:157-345 and block_pool.py
# ----------------------------------------------------------------------------------------------------------------
class FreeBlockQueue:
    """FIFO free list. Restates FreeKVCacheBlockQueue restricted to popleft/popleft_n/append_n (kv_cache_utils.py:
    206-345); its mid-queue ``remove`` is only reached through prefix-cache hits, which CompressLM disables."""

    def __init__(self, block_ids):
        self.q = deque(block_ids)

    @property
    def num_free_blocks(self):
        return len(self.q)

    def popleft(self):
        if not self.q:
            raise ValueError("No free blocks available")
        return self.q.popleft()

    def popleft_n(self, n):                                       # kv_cache_utils.py:246-276
        assert len(self.q) >= n
        return [self.q.popleft() for _ in range(n)]

    def append_n(self, blocks):                                   # kv_cache_utils.py:322-345
        self.q.extend(blocks)

    def order(self):
        return list(self.q)


class BlockPool:
    """Page pool: block_pool.py:160-176 (constructor, page 0 is the null block), :295-325 (get_new_blocks),
    :385-399 (free_blocks), :488-550 (copy_kv_slots).

    ``free_order`` lets a workload start from a fragmented free list (a permutation of pages 1..N-1) instead of
    id order; with ``free_order=None`` the construction is exactly the reference's."""

    def __init__(self, num_blocks, free_order=None):
        self.num_blocks = num_blocks
        self.ref_cnt = [0] * num_blocks
        self.free_queue = FreeBlockQueue(range(num_blocks))
        self.null_block = self.free_queue.popleft()               # block_pool.py:172-176
        if free_order is not None:
            free_order = [int(b) for b in free_order]
            if sorted(free_order) != list(range(1, num_blocks)):
                raise ValueError("free_order must be a permutation of pages 1..num_blocks-1")
            self.free_queue = FreeBlockQueue(free_order)

    def get_num_free_blocks(self):
        return self.free_queue.num_free_blocks

    def get_new_blocks(self, num_blocks):                         # block_pool.py:295-325
        if num_blocks > self.get_num_free_blocks():
            raise ValueError(f"Cannot get {num_blocks} free blocks from the pool")
        ret = self.free_queue.popleft_n(num_blocks)
        for b in ret:
            assert self.ref_cnt[b] == 0
            self.ref_cnt[b] += 1
        return ret

    def free_blocks(self, ordered_blocks):                        # block_pool.py:385-399
        blocks = list(ordered_blocks)
        for b in blocks:
            self.ref_cnt[b] -= 1
        self.free_queue.append_n([b for b in blocks if self.ref_cnt[b] == 0 and b != self.null_block])

    @staticmethod
    def copy_kv_slots(blocks, copy_operations, block_size):       # block_pool.py:488-550
        ops = []
        for src_slot, dst_slot in copy_operations:
            ops.append((blocks[src_slot // block_size], src_slot % block_size,
                        blocks[dst_slot // block_size], dst_slot % block_size))
        return ops


# ----------------------------------------------------------------------------------------------------------------
# third_party/vllm_overlay/vllm/v1/core/single_type_kv_cache_manager.py
# ----------------------------------------------------------------------------------------------------------------
class GroupManager:
    """One KV-cache group's per-request page lists (FullAttentionManager semantics, no prefix caching)."""

    def __init__(self, pool: BlockPool, block_size: int = PAGE):
        self.pool = pool
        self.block_size = block_size
        self.req_to_blocks: dict[str, list[int]] = {}

    def blocks(self, rid):
        return self.req_to_blocks.setdefault(rid, [])

    def get_num_blocks_to_allocate(self, rid, num_tokens):       # single_type_kv_cache_manager.py:66-99
        required = -(-num_tokens // self.block_size)
        return required - len(self.blocks(rid))

    def allocate_new_blocks(self, rid, num_tokens):              # single_type_kv_cache_manager.py:122-145
        req_blocks = self.blocks(rid)
        num_new = -(-num_tokens // self.block_size) - len(req_blocks)
        if num_new <= 0:
            return []
        new = self.pool.get_new_blocks(num_new)
        req_blocks.extend(new)
        return new

    def free(self, rid):                                          # single_type_kv_cache_manager.py:173-188
        req_blocks = self.req_to_blocks.pop(rid, [])
        self.pool.free_blocks(reversed(req_blocks))

    def compact_kv_cache_span(self, rid, start, end, num_active):  # single_type_kv_cache_manager.py:358-390
        if rid not in self.req_to_blocks:
            return 0, []
        if not 0 <= start < end <= num_active:
            raise ValueError(f"Invalid physical compaction span [{start}, {end}) for {num_active} active tokens")
        blocks = self.req_to_blocks[rid]
        if not blocks:
            return 0, []
        removed = end - start
        copy_operations = [(src, src - removed) for src in range(end, num_active)]
        ops = self.pool.copy_kv_slots(blocks, copy_operations, self.block_size)
        freed = self._truncate_compacted_blocks(blocks, num_active - removed)
        return freed, ops

    def _truncate_compacted_blocks(self, blocks, num_active):   # single_type_kv_cache_manager.py:392-420
        needed = (num_active + self.block_size - 1) // self.block_size
        freed, to_free = 0, []
        for i in range(needed, len(blocks)):
            if blocks[i] != self.pool.null_block:
                to_free.append(blocks[i])
                blocks[i] = self.pool.null_block
                freed += 1
        del blocks[needed:]
        if to_free:
            self.pool.free_blocks(reversed(to_free))
        return freed


@dataclass
class SpanRemovalResult:
    """vllm/v1/engine/__init__.py:203-213."""
    success: bool
    tokens_removed: int
    blocks_freed: int
    error_message: str | None = None


class RequestState:
    """The per-request fields the planner reads: num_computed_tokens and one span index per group
    (third_party/vllm_overlay/vllm/v1/request.py:263-321)."""

    def __init__(self, rid, num_groups):
        self.rid = rid
        self.num_computed_tokens = 0
        self.groups = [CompactedSpanIndex([]) for _ in range(num_groups)]

    def compacted_counts(self):
        return tuple(g.total_removed for g in self.groups)


class Planner:
    """Scheduler + KV-cache-manager bookkeeping of one pool shared by ``num_groups`` KV-cache groups."""

    def __init__(self, num_blocks, num_groups, block_size=PAGE, free_order=None, max_model_len=1 << 40):
        self.pool = BlockPool(num_blocks, free_order)
        self.block_size = block_size
        self.num_groups = num_groups
        self.max_model_len = max_model_len
        self.managers = [GroupManager(self.pool, block_size) for _ in range(num_groups)]
        self.requests: dict[str, RequestState] = {}
        self.pending_kv_copy_operations: dict[str, list[list[list[tuple]]]] = {}
        self.pending_block_table_truncations: dict[str, tuple[int, ...]] = {}

    def add_request(self, rid):
        self.requests[rid] = RequestState(rid, self.num_groups)

    def allocate_slots(self, rid, num_new_tokens):
        """kv_cache_manager.py:206-340 without prefix caching / lookahead / encoder tokens: per group
        need = min(computed + new, max_model_len) - compacted_g; abort (None) if the pool cannot cover the sum."""
        if num_new_tokens == 0:
            raise ValueError("num_new_tokens must be greater than 0")
        req = self.requests[rid]
        need = min(req.num_computed_tokens + num_new_tokens, self.max_model_len)
        per_group = [need - c for c in req.compacted_counts()]
        total = sum(m.get_num_blocks_to_allocate(rid, n) for m, n in zip(self.managers, per_group))
        if total > self.pool.get_num_free_blocks():
            return None
        return tuple(m.allocate_new_blocks(rid, n) for m, n in zip(self.managers, per_group))

    def free_request(self, rid):
        """kv_cache_coordinator free: every group frees its pages in reverse order, group by group."""
        for m in self.managers:
            m.free(rid)
        self.requests.pop(rid, None)
        self.pending_kv_copy_operations.pop(rid, None)
        self.pending_block_table_truncations.pop(rid, None)

    def block_ids(self, rid):
        return tuple(list(m.blocks(rid)) for m in self.managers)

    def mask_token_span(self, rid, start, end, groups=None) -> SpanRemovalResult:
        """scheduler.py:2060-2204."""
        req = self.requests.get(rid)
        if req is None:
            return SpanRemovalResult(False, 0, 0, f"Request {rid} not found")
        if start < 0 or end <= start:
            return SpanRemovalResult(False, 0, 0, "Invalid span: must have 0 <= start < end")
        if end > req.num_computed_tokens:
            return SpanRemovalResult(False, 0, 0,
                                     f"end_position ({end}) exceeds computed tokens ({req.num_computed_tokens})")
        new_span = (start, end)
        masked = end - start
        G = self.num_groups
        targets = list(range(G)) if groups is None else sorted(set(groups))
        plans = []
        for g in targets:
            if not 0 <= g < G:
                return SpanRemovalResult(False, 0, 0, f"KV cache group {g} out of range")
            if any(start < e and end > s for s, e in req.groups[g].spans):
                return SpanRemovalResult(False, 0, 0, f"Cannot compact an already-removed token span (group {g})")
            ps = req.groups[g].logical_to_physical(start)
            pe = req.groups[g].logical_to_physical(end)
            if pe - ps != masked:
                return SpanRemovalResult(False, 0, 0,
                                         f"Logical span does not map to one active physical span (group {g})")
            active = req.num_computed_tokens - req.groups[g].total_removed
            if active == masked:
                return SpanRemovalResult(False, 0, 0, "Cannot compact: all tokens would be removed")
            plans.append((g, ps, pe, active))
        total_freed = 0
        for g, ps, pe, active in plans:
            freed, ops = self.managers[g].compact_kv_cache_span(rid, ps, pe, active)
            total_freed += freed
            if ops:
                per_group = self.pending_kv_copy_operations.setdefault(rid, [[] for _ in range(G)])
                per_group[g].append(ops)
            req.groups[g] = CompactedSpanIndex(merge_spans(req.groups[g].spans + [new_span]))
        self.pending_block_table_truncations[rid] = tuple(len(m.blocks(rid)) for m in self.managers)
        return SpanRemovalResult(True, masked, total_freed)

    def apply_events(self, rows) -> None:
        """Scheduler events in the native planner's event-row format (kind, rid, a, b, group_mask, 0): 0 add,
        1 schedule a tokens (allocate, then count them computed), 2 mask [a, b) in the groups of group_mask (< 0:
        all), 3 free, 4 take (drop) the step outputs. A rejected allocation or span raises."""
        for kind, rid, a, b, gm, _ in np.asarray(rows, np.int64).tolist():
            if kind == 0:
                self.add_request(rid)
            elif kind == 1:
                if self.allocate_slots(rid, a) is None:
                    raise RuntimeError("oracle pool exhausted")
                self.requests[rid].num_computed_tokens += a
            elif kind == 2:
                groups = None if gm < 0 else [g for g in range(self.num_groups) if (gm >> g) & 1]
                res = self.mask_token_span(rid, a, b, groups)
                if not res.success:
                    raise RuntimeError(res.error_message)
            elif kind == 3:
                self.free_request(rid)
            else:
                self.take_step_outputs()

    def take_step_outputs(self):
        """What the next SchedulerOutput carries (output.py:221-225), then cleared."""
        ops, trunc = self.pending_kv_copy_operations, self.pending_block_table_truncations
        self.pending_kv_copy_operations, self.pending_block_table_truncations = {}, {}
        return ops, trunc

    def physical_positions(self, rid, logical_positions):
        """gpu_model_runner.py:1585-1590: phys_g = logical - compacted_tokens[req, g]."""
        req = self.requests[rid]
        lp = np.asarray(logical_positions, dtype=np.int64)
        return [lp - c for c in req.compacted_counts()]

    def seq_lens(self, rid, num_scheduled):
        """gpu_model_runner.py:1674-1682: seq_len_g = computed - compacted_g + scheduled (before the step's
        computed-token update, i.e. with ``num_computed_tokens`` excluding the scheduled tokens)."""
        req = self.requests[rid]
        return [req.num_computed_tokens - c + num_scheduled for c in req.compacted_counts()]


def slot_mapping(block_ids, positions, block_size=PAGE):
    """block_table.py:186-197 (non-CP): slot = table[pos // block_size] * block_size + pos % block_size."""
    positions = np.asarray(positions, dtype=np.int64)
    table = np.asarray(block_ids, dtype=np.int64)
    return table[positions // block_size] * block_size + positions % block_size


def execute_kv_copy_operations(kv_copy_operations, layer_caches_by_group):
    """gpu_model_runner.py:1147-1176 and :1194-1224.

    ``kv_copy_operations``: request id -> per group -> ordered batches of (src_block, src_off, dst_block, dst_off).
    For every group, batch b of every request is merged and applied with gather-then-scatter semantics to each
    layer cache of that group (numpy arrays shaped [num_blocks, 2, block_size, ...])."""
    for gid, caches in enumerate(layer_caches_by_group):
        batches = [ops[gid] for ops in kv_copy_operations.values() if gid < len(ops)]
        num_batches = max((len(b) for b in batches), default=0)
        for b in range(num_batches):
            all_ops = []
            for req_batches in batches:
                if b < len(req_batches):
                    all_ops.extend(req_batches[b])
            if not all_ops:
                continue
            op = np.asarray(all_ops, dtype=np.int64)
            for cache in caches:
                source = cache[op[:, 0], :, op[:, 1]].copy()
                cache[op[:, 2], :, op[:, 3]] = source
