"""Per-head packed code pages: the storage and attention of per-head quota schedules on the MI355X kernels.

Mirrors the reference's packed KV sidecar (third_party/vllm_overlay/vllm/v1/worker/compresslm_packed_kv.py):
``PackedKVLayout`` (:12-155) is the static ``K[layer, kv_head]`` layout of one compressed block with the same API and
errors; ``PackedKVSidecar`` (:214-741) keeps the packed pages and attends them. Where the reference holds one small
torch tensor per (request, layer, block) and attends with gathers and einsums, here each layer has one device pool
``[pool_pages, 2, rows_l, 128]`` (rows_l = sum of the layer's head quotas); a request owns a list of pool pages (one
per captured block, the same page id in every layer). ``capture`` copies a closed block's code rows from every
layer's paged cache in one launch (``abkv_packed_capture``); attention runs ``abkv_decode_attn_packed`` when every
active request decodes one token and ``abkv_paged_prefill_attn_packed`` otherwise (prompt chunks: causal over the
paged rows; code steps: non-causal, paged keys ``< prefix_len + q_h`` for KV head h), the side rows of head h
visible to every query of the request in both.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import numpy as np
import torch

from . import ops

HEADS_KV = ops.HEADS_KV


@dataclass(frozen=True)
class PackedKVLayout:
    """Static ``K[layer, kv_head]`` layout for one compressed block (compresslm_packed_kv.py:12-155)."""

    quotas: tuple[tuple[int, ...], ...]
    k_max: int

    def __post_init__(self) -> None:
        if self.k_max <= 0:
            raise ValueError("packed KV k_max must be positive")
        if not self.quotas or not self.quotas[0]:
            raise ValueError("packed KV quotas must be a non-empty 2D schedule")
        num_heads = len(self.quotas[0])
        for layer, row in enumerate(self.quotas):
            if len(row) != num_heads:
                raise ValueError("packed KV quota rows must have equal length; "
                                 f"layer 0 has {num_heads}, layer {layer} has {len(row)}")
            for head, quota in enumerate(row):
                if not 0 < quota <= self.k_max:
                    raise ValueError(f"packed KV quota[{layer}][{head}]={quota} must be in [1, {self.k_max}]")

    @classmethod
    def from_schedule(cls, schedule: Sequence[Sequence[int]] | None, *, num_layers: int, num_kv_heads: int,
                      k_max: int) -> "PackedKVLayout":
        if num_layers <= 0 or num_kv_heads <= 0:
            raise ValueError("packed KV model dimensions must be positive")
        if schedule:
            quotas = tuple(tuple(int(v) for v in row) for row in schedule)
        else:
            quotas = tuple((int(k_max),) * num_kv_heads for _ in range(num_layers))
        if len(quotas) != num_layers:
            raise ValueError(f"packed KV schedule has {len(quotas)} layers; model has {num_layers}")
        if any(len(row) != num_kv_heads for row in quotas):
            widths = sorted(set(len(row) for row in quotas))
            raise ValueError(f"packed KV schedule row widths {widths} do not match model num_kv_heads={num_kv_heads}")
        return cls(quotas=quotas, k_max=int(k_max))

    @property
    def num_layers(self) -> int:
        return len(self.quotas)

    @property
    def num_kv_heads(self) -> int:
        return len(self.quotas[0])

    @property
    def offsets(self) -> tuple[tuple[int, ...], ...]:
        return tuple(tuple(int(x) for x in np.concatenate([[0], np.cumsum(row)])) for row in self.quotas)

    @property
    def packed_slots_per_layer(self) -> tuple[int, ...]:
        return tuple(sum(row) for row in self.quotas)

    @property
    def packed_slots(self) -> int:
        return sum(self.packed_slots_per_layer)

    @property
    def dense_slots(self) -> int:
        return self.num_layers * self.num_kv_heads * self.k_max

    @property
    def storage_ratio(self) -> float:
        return self.packed_slots / self.dense_slots

    def bytes_per_block(self, *, head_size: int, element_size: int) -> int:
        if head_size <= 0 or element_size <= 0:
            raise ValueError("head_size and element_size must be positive")
        return 2 * self.packed_slots * head_size * element_size

    def dense_bytes_per_block(self, *, head_size: int, element_size: int) -> int:
        if head_size <= 0 or element_size <= 0:
            raise ValueError("head_size and element_size must be positive")
        return 2 * self.dense_slots * head_size * element_size

    def pack_layer(self, layer: int, dense: torch.Tensor) -> torch.Tensor:
        """Pack ``[2, K_max, H_kv, D]`` into ``[2, sum_h K_lh, D]`` (head h's first K_lh rows, heads in order)."""
        expected = (2, self.k_max, self.num_kv_heads)
        if dense.ndim != 4 or tuple(dense.shape[:3]) != expected:
            raise ValueError(f"dense layer KV must start with shape {expected}; got {tuple(dense.shape)}")
        return torch.cat([dense[:, :q, h, :] for h, q in enumerate(self.quotas[layer])], dim=1).contiguous()

    def unpack_layer(self, layer: int, packed: torch.Tensor, *, fill_value: float = 0.0) -> torch.Tensor:
        """Expand a packed layer page to ``[2, K_max, H_kv, D]`` (rows past a head's quota hold fill_value)."""
        expected_slots = self.packed_slots_per_layer[layer]
        if packed.ndim != 3 or packed.shape[0] != 2:
            raise ValueError("packed layer KV must have shape [2, packed_slots, head_size]")
        if packed.shape[1] != expected_slots:
            raise ValueError(f"packed layer {layer} has {packed.shape[1]} slots; expected {expected_slots}")
        dense = packed.new_full((2, self.k_max, self.num_kv_heads, packed.shape[-1]), fill_value)
        off = self.offsets[layer]
        for h, q in enumerate(self.quotas[layer]):
            dense[:, :q, h, :] = packed[:, off[h]: off[h + 1], :]
        return dense


class PackedKVSidecar:
    """Device pools of packed pages and the attention consumer over them (compresslm_packed_kv.py:214-741).

    ``kv_caches``: per layer the paged cache [P, 2, 16, 8, 128] bf16 the captures read (the reference reads
    ``attention_layers[l].kv_cache[0]``; layer objects with that attribute are accepted too). ``pool_pages`` bounds
    the captured blocks alive at once; ``max_pages_per_request`` bounds one request's (<= 2048).
    """

    def __init__(self, layout: PackedKVLayout, kv_caches: Sequence, *, block_size: int = 16,
                 pool_pages: int = 4096, max_pages_per_request: int = 512, device=None) -> None:
        if len(kv_caches) != layout.num_layers:
            raise ValueError(f"received {len(kv_caches)} attention layers for {layout.num_layers}-layer packed layout")
        if layout.num_kv_heads != HEADS_KV:
            raise ValueError(f"the kernels serve {HEADS_KV} KV heads; layout has {layout.num_kv_heads}")
        if int(block_size) != ops.PAGE:
            raise ValueError(f"the kernels serve block_size {ops.PAGE}")
        if not 0 < max_pages_per_request <= 2048:
            raise ValueError("max_pages_per_request must be in [1, 2048]")
        self.layout = layout
        self.block_size = int(block_size)
        caches = [getattr(c, "kv_cache", c) for c in kv_caches]
        self.kv_caches = [c[0] if isinstance(c, (list, tuple)) else c for c in caches]
        self.device = torch.device(device) if device is not None else self.kv_caches[0].device
        self.pool_pages = int(pool_pages)
        self.max_pages_per_request = int(max_pages_per_request)
        self.pools = [torch.empty((self.pool_pages, 2, rows, ops.HEAD_DIM), dtype=torch.bfloat16, device=self.device)
                      for rows in layout.packed_slots_per_layer]
        q = np.asarray(layout.quotas, dtype=np.int32)
        self._rows_dev = torch.from_numpy(np.asarray(layout.packed_slots_per_layer, dtype=np.int32)).to(self.device)
        self._quota_dev = torch.from_numpy(np.ascontiguousarray(q)).to(self.device)
        self._free = list(range(self.pool_pages - 1, -1, -1))
        self.pages: dict[str, list[int]] = {}
        self.active_request_ids: tuple[str, ...] = ()
        self.common_attn_metadata = None
        self._step_tables = None

    # -- bookkeeping --------------------------------------------------------------------------------------------
    def set_active_request_ids(self, request_ids: Sequence[str]) -> None:
        self.active_request_ids = tuple(request_ids)
        self._step_tables = None

    def set_common_attn_metadata(self, metadata) -> None:
        self.common_attn_metadata = metadata
        self._step_tables = None

    def free(self, request_id: str) -> None:
        for p in self.pages.pop(request_id, []):
            self._free.append(p)
        self._step_tables = None

    @property
    def allocated_bytes(self) -> int:
        used = sum(len(v) for v in self.pages.values())
        return used * self.layout.bytes_per_block(head_size=ops.HEAD_DIM, element_size=2)

    def request_pages(self, request_id: str) -> list[int]:
        return list(self.pages.get(request_id, []))

    # -- capture ------------------------------------------------------------------------------------------------
    def capture(self, request_id: str, *, physical_start: int, physical_end: int, block_ids) -> None:
        """Pack the k_max code rows ``[physical_start, physical_end)`` of every layer (block_ids: the request's
        page table row in the paged caches)."""
        self.capture_many([(request_id, physical_start, physical_end, block_ids)])

    def capture_many(self, captures) -> None:
        """Several captures ``(request_id, physical_start, physical_end, block_ids)`` in one launch."""
        if not captures:
            return
        width = max(len(c[3]) for c in captures)
        table = np.zeros((len(captures), max(width, 1)), dtype=np.int32)
        starts = np.zeros(len(captures), dtype=np.int32)
        dst = np.zeros(len(captures), dtype=np.int32)
        for i, (rid, start, end, block_ids) in enumerate(captures):
            if end - start != self.layout.k_max:
                raise ValueError("packed KV capture must contain exactly k_max code rows; "
                                 f"got {end - start}, expected {self.layout.k_max}")
            ids = np.asarray(list(block_ids), dtype=np.int64)
            if start < 0 or -(-end // self.block_size) > ids.size:
                raise ValueError(f"packed KV capture span [{start}, {end}) exceeds the request's page table")
            owned = self.pages.setdefault(rid, [])
            if len(owned) >= self.max_pages_per_request:
                raise RuntimeError(f"request {rid} holds {len(owned)} packed pages (max {self.max_pages_per_request})")
            if not self._free:
                raise RuntimeError("packed KV pool exhausted")
            page = self._free.pop()
            owned.append(page)
            table[i, : ids.size] = ids
            starts[i] = start
            dst[i] = page
        dev = self.device
        meta = torch.from_numpy(np.concatenate([starts, dst])).to(dev)
        n = len(captures)
        ops.packed_capture(self.kv_caches, self.pools, self._rows_dev, self._quota_dev,
                           torch.from_numpy(table).to(dev), meta[:n], meta[n:])
        self._step_tables = None

    # -- attention ----------------------------------------------------------------------------------------------
    def _tables(self, request_ids):
        if self._step_tables is not None and self._step_tables[0] == request_ids:
            return self._step_tables[1:]
        counts = np.asarray([len(self.pages.get(r, [])) for r in request_ids], dtype=np.int32)
        width = max(1, int(counts.max()) if counts.size else 1)
        table = np.zeros((len(request_ids), width), dtype=np.int32)
        for i, r in enumerate(request_ids):
            ids = self.pages.get(r, [])
            table[i, : len(ids)] = ids
        dev = self.device
        out = (torch.from_numpy(table).to(dev), torch.from_numpy(counts).to(dev), int(counts.max(initial=0)))
        self._step_tables = (request_ids,) + out
        return out

    def attend(self, layer_index: int, query: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor,
               query_start_loc, seq_lens, causal, output: torch.Tensor, request_ids=None,
               seq_lens_dev: torch.Tensor | None = None, scale: float | None = None, lse=None,
               excluded=None) -> torch.Tensor:
        """Attention of one layer for a batch of requests: paged rows (``block_table``, ``seq_lens`` physical rows
        after this step's tokens, host ``query_start_loc``) plus each request's packed side rows. ``causal``: one
        flag for the batch or one per request (a non-causal request is a code step of exactly k_max queries).
        ``excluded``: None or per request the physical paged rows a code step must not see (its block's static
        tail, compresslm_packed_kv.py:725-729)."""
        rids = tuple(self.active_request_ids if request_ids is None else request_ids)
        qsl = np.asarray(query_start_loc, dtype=np.int64)
        sl = np.asarray(seq_lens, dtype=np.int64)
        B = sl.size
        if len(rids) != B or qsl.size != B + 1:
            raise RuntimeError("packed KV attention needs one request id per request")
        nq = np.diff(qsl)
        cz = np.broadcast_to(np.asarray(causal, dtype=bool), (B,))
        for r in range(B):
            if not cz[r] and nq[r] != self.layout.k_max:
                raise RuntimeError("packed KV noncausal step must contain exactly "
                                   f"k_max={self.layout.k_max} code queries; got {int(nq[r])}")
        table, count, max_packed = self._tables(rids)
        quotas = self.layout.quotas[layer_index]
        pool = self.pools[layer_index]
        scale = ops.default_scale() if scale is None else float(scale)
        T = int(qsl[-1])
        if T == 0:
            return output
        if bool(np.all(nq == 1)) and bool(np.all(cz)):
            if seq_lens_dev is None:
                seq_lens_dev = torch.from_numpy(sl.astype(np.int32)).to(query.device)
            max_pages = max(1, int(-(-sl.max() // ops.PAGE)))
            ops.decode_attention_packed(query[:B], kv_cache, block_table, seq_lens_dev, pool, quotas, table, count,
                                        scale, max_pages=min(max_pages, block_table.shape[1]),
                                        max_packed=max_packed, out=output[:B], lse=lse,
                                        split_pages=ops.auto_split_pages(sl))
            return output
        kv_start = sl - nq
        ops.paged_prefill_attention_packed(query[:T], kv_cache, block_table, qsl, kv_start, sl, cz, pool, quotas,
                                           table, count, max_packed, scale=scale, out=output[:T], lse=lse,
                                           head_quota_dev=self._quota_dev[layer_index], excluded=excluded)
        return output

    def override_attention(self, *, layer_index: int, layer, query: torch.Tensor, kv_cache: torch.Tensor,
                           attn_metadata, output: torch.Tensor) -> None:
        """The overlay hook's consumer (compresslm_packed_kv.py:286-484): metadata from
        ``set_common_attn_metadata`` (fields ``query_start_loc``(``_cpu``), ``seq_lens``(``_cpu``),
        ``block_table``(``_tensor``), ``causal``) or ``attn_metadata`` itself."""
        if not self.active_request_ids:
            return
        if query.dtype != torch.bfloat16:
            raise RuntimeError(f"packed KV attention runs bf16; got {query.dtype}")
        common = self.common_attn_metadata if self.common_attn_metadata is not None else attn_metadata
        if common is None:
            raise RuntimeError("packed KV common attention metadata is absent")
        qsl = getattr(common, "query_start_loc_cpu", None)
        qsl = getattr(common, "query_start_loc") if qsl is None else qsl
        sl = getattr(common, "_seq_lens_cpu", None)
        sl = getattr(common, "seq_lens") if sl is None else sl
        bt = getattr(common, "block_table_tensor", None)
        bt = getattr(common, "block_table") if bt is None else bt
        qsl = np.asarray(qsl.cpu() if torch.is_tensor(qsl) else qsl, dtype=np.int64)
        sl = np.asarray(sl.cpu() if torch.is_tensor(sl) else sl, dtype=np.int64)
        n = len(self.active_request_ids)
        scale = getattr(getattr(layer, "impl", None), "scale", None)
        self.attend(layer_index, query.view(-1, ops.HEADS_Q, ops.HEAD_DIM), kv_cache, bt, qsl[: n + 1], sl[:n],
                    bool(getattr(common, "causal", True)), output.view(-1, ops.HEADS_Q, ops.HEAD_DIM), scale=scale)


def maybe_override_attention(layer, query: torch.Tensor, kv_cache: torch.Tensor, attn_metadata,
                             output: torch.Tensor) -> None:
    """The overlay hook (compresslm_packed_kv.py:744-761): a layer carrying a sidecar attends through it."""
    sidecar = getattr(layer, "_compresslm_packed_sidecar", None)
    if sidecar is None or attn_metadata is None:
        return
    sidecar.override_attention(layer_index=layer._compresslm_packed_layer_index, layer=layer, query=query,
                               kv_cache=kv_cache, attn_metadata=attn_metadata, output=output)
