"""Attention backend over the abridged paged cache: the drop-in for the serving attention call.

Mirrors the backend contract the overlay runs on (vLLM ``Attention.forward`` -> backend
``forward(layer, query, key, value, kv_cache, attn_metadata, output)``; metadata fields from
``CommonAttentionMetadata`` as built at third_party/vllm_overlay/vllm/v1/worker/gpu_model_runner.py:1872-1887,
2244-2266) and the overlay's in-place override hook ``maybe_override_attention(layer, query, kv_cache,
attn_metadata, output)`` (third_party/vllm_overlay/vllm/v1/worker/compresslm_packed_kv.py:744-761).

One metadata object describes one KV-cache group on one step (each group has its own physical lengths and page
table, gpu_model_runner.py:1672-1682). A step's batch is ordered decodes first (one query token each, the
reorder FlashInfer applies with decode threshold 1) and then multi-token requests:

* decode requests -> ``abkv_decode_attn`` (split-KV decode; graph-capturable, fixed workspace), called as the
  custom op ``torch.ops.abridgekv.decode_attn`` so compiled callers keep it as one node;
* prompt chunks -> ``abkv_paged_prefill_attn`` causal;
* CompressLM code-step requests -> ``abkv_paged_prefill_attn`` non-causal with the key limit
  ``code_start + quota``: the physical-quota code mask of gpu_model_runner.py:2042-2107 (all resident rows, the
  block's own code slots ``>= quota`` hidden; compresslm_masks.py:165-239) expressed as a per-request limit, and with
  a retained tail the block's own tail rows hidden as a per-request excluded range (:2086-2094).

New K/V rows are written by ``abkv_kv_append`` (``torch.ops.abridgekv.kv_append``) before attention
(``reshape_and_cache`` semantics: slot < 0 skips).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from . import ops
from . import torch_ops  # noqa: F401  (torch.ops.abridgekv.*)

NOT_CODE = -1


@dataclass
class AbridgeAttentionMetadata:
    """One KV-cache group's view of one step.

    ``query_start_loc`` [B+1] and ``seq_lens`` [B] (physical rows of the group after this step's tokens) are host
    int arrays; ``block_table`` [B, W] int32, ``slot_mapping`` [T] int64 and ``seq_lens_dev`` [B] int32 live on the
    GPU. ``code_key_limit`` [B] holds, for a code-step request, the physical key limit (code start + the group's
    quota) and ``NOT_CODE`` for every other request; ``code_excluded`` [B, 2] the physical rows a code-step request
    must not see (its block's retained tail; an empty range otherwise), or None; ``code_causal`` [B] bool, for a
    code-step request whose code rows see their own block's codes causally (``pause_xattn="causal"`` of the
    generator; the serving path's code steps are bidirectional), or None. ``num_decodes`` leading requests have one
    query token.
    """
    query_start_loc: np.ndarray
    seq_lens: np.ndarray
    block_table: torch.Tensor
    slot_mapping: torch.Tensor
    seq_lens_dev: torch.Tensor
    num_decodes: int
    code_key_limit: np.ndarray
    max_decode_pages: int
    workspace: torch.Tensor | None = None
    causal: bool = True
    split_pages: int = ops.DEFAULT_SPLIT_PAGES
    code_excluded: np.ndarray | None = None
    code_causal: np.ndarray | None = None

    @property
    def num_reqs(self) -> int:
        return int(self.seq_lens.size)

    @property
    def num_decode_tokens(self) -> int:
        return int(self.query_start_loc[self.num_decodes])

    @property
    def num_actual_tokens(self) -> int:
        return int(self.query_start_loc[-1])


def code_step_key_limits(query_start_loc, seq_lens, code_spans, group_quota: int, num_code_tokens: int) -> np.ndarray:
    """Per-request key limits of a code step in one group (physical-quota masks, gpu_model_runner.py:2042-2107).

    ``code_spans[r]`` is the physical ``(start, end)`` of the block being coded (``CompressLMProcessor.
    code_physical_spans`` of the group, restricted to that block) or ``None`` for a request that is not coding. The
    span must be exactly the request's query rows (the code step's queries are the block's K code rows). A request
    sees every row before its code span and the first ``min(quota, K)`` rows of it.
    """
    qsl = np.asarray(query_start_loc, dtype=np.int64)
    sl = np.asarray(seq_lens, dtype=np.int64)
    out = np.full(sl.size, NOT_CODE, dtype=np.int64)
    for r, span in enumerate(code_spans):
        if span is None:
            continue
        start, end = int(span[0]), int(span[1])
        q_len = int(qsl[r + 1] - qsl[r])
        if not (0 <= start < end <= sl[r]):
            raise RuntimeError(f"code span {(start, end)} outside seq_len={int(sl[r])} (request {r})")
        if end != sl[r] or end - start != q_len:
            raise RuntimeError(f"code span {(start, end)} must be the request's {q_len} query rows ending at "
                               f"seq_len={int(sl[r])} (request {r})")
        out[r] = start + min(int(group_quota), int(num_code_tokens), end - start)
    return out


def code_step_excluded_ranges(code_spans, excluded_ranges, query_start_loc, seq_lens) -> np.ndarray | None:
    """Per-request excluded key ranges [B, 2] of a code step in one group (the block's own retained tail,
    ``CompressLMProcessor.code_excluded_physical_ranges`` of the group), checked as the worker checks them
    (gpu_model_runner.py:2086-2091: ``0 <= start < end <= seq_len - query_len``); None when no request has one."""
    qsl = np.asarray(query_start_loc, dtype=np.int64)
    sl = np.asarray(seq_lens, dtype=np.int64)
    out = np.zeros((sl.size, 2), dtype=np.int64)
    any_range = False
    for r, ex in enumerate(excluded_ranges):
        if ex is None:
            continue
        if code_spans[r] is None:
            raise RuntimeError(f"request {r} has an excluded range but is not coding")
        start, end = int(ex[0]), int(ex[1])
        if not 0 <= start < end <= sl[r] - (qsl[r + 1] - qsl[r]):
            raise RuntimeError(f"invalid CompressLM code exclusion range {(start, end)} for "
                               f"query_len={int(qsl[r + 1] - qsl[r])}, seq_len={int(sl[r])}")
        out[r] = (start, end)
        any_range = True
    return out if any_range else None


def key_ranges_from_custom_mask(mask: torch.Tensor, query_start_loc, seq_lens):
    """Turn a flat custom mask of the reference's format (row-major per-request ``q_len x seq_len`` blocks,
    compresslm_masks.py:165-239) into per-request ``(key_limit, causal, excluded)``.

    Accepts exactly the masks this backend can run: per request, either every query row sees the same set
    ``[0, L)`` minus at most one contiguous range ``[a, b)`` inside it (a code step; the range is its block's static
    tail) or row i sees ``[0, seq_len - q_len + i]`` (a causal chunk). ``excluded`` is None when no request hides a
    range, else [B, 2] (an empty range for the others). Any other mask raises ``RuntimeError``: the kernels keep no
    dense mask.
    """
    m = mask.detach().to("cpu", torch.bool).numpy().reshape(-1)
    qsl = np.asarray(query_start_loc, dtype=np.int64)
    sl = np.asarray(seq_lens, dtype=np.int64)
    B = sl.size
    limits = np.zeros(B, dtype=np.int64)
    causal = np.zeros(B, dtype=bool)
    excluded = np.zeros((B, 2), dtype=np.int64)
    at = 0
    for r in range(B):
        q_len, s_len = int(qsl[r + 1] - qsl[r]), int(sl[r])
        block = m[at: at + q_len * s_len]
        at += q_len * s_len
        if block.size != q_len * s_len:
            raise RuntimeError("custom mask is shorter than sum(q_len * seq_len)")
        if q_len == 0:
            limits[r] = s_len
            continue
        block = block.reshape(q_len, s_len)
        col = np.arange(s_len)
        if np.all(block == block[0]):
            row = block[0]
            lim = int(np.flatnonzero(row)[-1]) + 1 if row.any() else 0
            gap = np.flatnonzero(~row[:lim])
            if gap.size and gap[-1] - gap[0] + 1 != gap.size:
                raise RuntimeError(f"custom mask of request {r} hides more than one key range")
            limits[r] = lim
            if gap.size:
                excluded[r] = (gap[0], gap[-1] + 1)
            continue
        counts = block.sum(axis=1)
        if not np.array_equal(block, col[None, :] < counts[:, None]):
            raise RuntimeError(f"custom mask of request {r} is not a per-row key prefix")
        if np.array_equal(counts, s_len - q_len + 1 + np.arange(q_len)):
            limits[r], causal[r] = s_len, True
        else:
            raise RuntimeError(f"custom mask of request {r} is neither a shared key limit nor causal")
    if at != m.size:
        raise RuntimeError("custom mask is longer than sum(q_len * seq_len)")
    return limits, causal, (excluded if excluded[:, 1].any() else None)


def limits_from_custom_mask(mask: torch.Tensor, query_start_loc, seq_lens) -> tuple[np.ndarray, np.ndarray]:
    """:func:`key_ranges_from_custom_mask` for masks without an excluded range: per-request ``(key_limit, causal)``;
    a mask that hides a range inside a request's keys raises ``RuntimeError``."""
    limits, causal, excluded = key_ranges_from_custom_mask(mask, query_start_loc, seq_lens)
    if excluded is not None:
        r = int(np.flatnonzero(excluded[:, 1])[0])
        raise RuntimeError(f"custom mask of request {r} is not a per-row key prefix")
    return limits, causal


@dataclass
class AbridgeMetadataBuilder:
    """Builds per-group metadata once per step and owns the fixed decode workspace (sized for ``max_num_seqs``
    requests of up to ``max_pages`` pages, so decode launches never allocate and can be graph-captured)."""
    max_num_seqs: int
    max_pages: int
    device: torch.device | str = "cuda"
    split_pages: int | None = None          # None: per step, ops.auto_split_pages of the decode requests' rows
    _workspace: torch.Tensor | None = field(default=None, init=False, repr=False)

    def workspace(self) -> torch.Tensor:
        if self._workspace is None:
            sp = min(self.split_pages or ops.DEFAULT_SPLIT_PAGES, ops.DEFAULT_SPLIT_PAGES)
            self._workspace = ops.decode_workspace(self.max_num_seqs, self.max_pages, sp, device=self.device)
        return self._workspace

    def build(self, query_start_loc, seq_lens, block_table: torch.Tensor, slot_mapping: torch.Tensor | None = None,
              code_key_limit=None, seq_lens_dev: torch.Tensor | None = None, positions: torch.Tensor | None = None,
              compacted: torch.Tensor | None = None, code_excluded=None, code_causal=None) -> AbridgeAttentionMetadata:
        """One group's metadata of a step. ``slot_mapping`` [T] int64 (device), or None to compute it on the device
        from ``positions`` [T] int64 (the tokens' logical positions) and ``compacted`` [B] int32 (tokens the group
        removed per request): slot = table[r][p // 16] * 16 + p % 16 with p = position - compacted[r]
        (gpu_model_runner.py:1579-1661, block_table.py:186-197). ``code_excluded``: None, or [B, 2] physical key
        ranges the code-step requests must not see (:func:`code_step_excluded_ranges`). ``code_causal``: None, or [B]
        flags of code-step requests whose rows see their own codes causally (up to their own row and the key
        limit)."""
        qsl = np.asarray(query_start_loc, dtype=np.int64)
        sl = np.asarray(seq_lens, dtype=np.int64)
        B = sl.size
        if qsl.size != B + 1 or qsl[0] != 0 or np.any(np.diff(qsl) < 0):
            raise RuntimeError("query_start_loc must be a [B+1] prefix sum starting at 0")
        qlen = np.diff(qsl)
        if np.any(qlen > sl):
            raise RuntimeError("query_len exceeds seq_len")
        if B > self.max_num_seqs:
            raise RuntimeError(f"{B} requests exceed max_num_seqs={self.max_num_seqs}")
        limits = (np.full(B, NOT_CODE, dtype=np.int64) if code_key_limit is None
                  else np.asarray(code_key_limit, dtype=np.int64).reshape(B))
        decode = (qlen == 1) & (limits == NOT_CODE)
        nd = int(np.argmin(decode)) if not decode.all() else B
        if decode[nd:].any():
            raise RuntimeError("decode requests must precede multi-token and code-step requests in the batch")
        W = block_table.shape[1]
        if np.any(sl > W * ops.PAGE):
            raise RuntimeError("seq_len exceeds the block table width")
        code = limits != NOT_CODE
        if np.any(code & ((limits < sl - qlen) | (limits > sl))):
            raise RuntimeError("code key limit must lie within the request's own query rows")
        if code_excluded is not None:
            code_excluded = np.asarray(code_excluded, dtype=np.int64).reshape(B, 2)
            has = code_excluded[:, 1] > code_excluded[:, 0]
            if np.any(has & ~code):
                raise RuntimeError("only code-step requests may carry an excluded key range")
            if np.any(has & ((code_excluded[:, 0] < 0) | (code_excluded[:, 1] > sl - qlen))):
                raise RuntimeError("an excluded key range must lie before the request's own query rows")
            if not has.any():
                code_excluded = None
        if code_causal is not None:
            code_causal = np.asarray(code_causal, dtype=bool).reshape(B)
            if np.any(code_causal & ~code):
                raise RuntimeError("only code-step requests may be causal code steps")
        max_pages = int(-(-sl[:nd].max() // ops.PAGE)) if nd else 0
        if max_pages > self.max_pages:
            raise RuntimeError(f"decode needs {max_pages} pages > max_pages={self.max_pages}")
        if seq_lens_dev is None:
            seq_lens_dev = torch.from_numpy(sl.astype(np.int32)).to(block_table.device)
        if slot_mapping is None:
            if positions is None:
                raise RuntimeError("build needs slot_mapping or the tokens' logical positions")
            req_idx = torch.from_numpy(np.repeat(np.arange(B, dtype=np.int32), qlen)).to(block_table.device)
            slot_mapping = ops.slot_mapping(req_idx, positions, block_table, compacted=compacted)
        return AbridgeAttentionMetadata(query_start_loc=qsl, seq_lens=sl, block_table=block_table,
                                        slot_mapping=slot_mapping, seq_lens_dev=seq_lens_dev, num_decodes=nd,
                                        code_key_limit=limits, code_excluded=code_excluded, code_causal=code_causal,
                                        max_decode_pages=max(max_pages, 1),
                                        workspace=self.workspace() if nd else None,
                                        split_pages=self.split_pages or (ops.auto_split_pages(sl[:nd]) if nd
                                                                         else ops.DEFAULT_SPLIT_PAGES))


class AbridgeAttentionImpl:
    """Backend implementation for one attention layer (32 query heads, 8 KV heads, head size 128, bf16)."""

    def __init__(self, num_heads: int = ops.HEADS_Q, head_size: int = ops.HEAD_DIM, scale: float | None = None,
                 num_kv_heads: int = ops.HEADS_KV, kv_cache_dtype: str = "auto"):
        if (num_heads, head_size, num_kv_heads) != (ops.HEADS_Q, ops.HEAD_DIM, ops.HEADS_KV):
            raise NotImplementedError(f"kernels are built for {ops.HEADS_Q} q heads, {ops.HEADS_KV} KV heads, "
                                      f"head size {ops.HEAD_DIM}")
        if kv_cache_dtype not in ("auto", "bfloat16"):
            raise NotImplementedError("kv cache dtype must be bf16")
        self.num_heads, self.head_size, self.num_kv_heads = num_heads, head_size, num_kv_heads
        self.scale = ops.default_scale() if scale is None else float(scale)

    def forward(self, layer, query: torch.Tensor, key: torch.Tensor | None, value: torch.Tensor | None,
                kv_cache: torch.Tensor, attn_metadata: AbridgeAttentionMetadata | None,
                output: torch.Tensor | None = None, output_lse: torch.Tensor | None = None) -> torch.Tensor:
        """Append this step's K/V rows, then attend. query [T, 32*128] or [T, 32, 128]; output likewise (written in
        place and returned). ``attn_metadata`` None (profiling run) leaves the output untouched."""
        T = query.shape[0]
        q = query.view(T, self.num_heads, self.head_size)
        if output is None:
            output = torch.empty_like(query)
        if attn_metadata is None:
            return output
        md = attn_metadata
        if key is not None:
            n = md.num_actual_tokens
            torch.ops.abridgekv.kv_append(key.view(-1, self.num_kv_heads, self.head_size)[:n],
                                          value.view(-1, self.num_kv_heads, self.head_size)[:n], md.slot_mapping[:n],
                                          kv_cache)
        self.attend(q, kv_cache, md, output.view(T, self.num_heads, self.head_size), output_lse)
        return output

    def attend(self, q: torch.Tensor, kv_cache: torch.Tensor, md: AbridgeAttentionMetadata, out: torch.Tensor,
               lse: torch.Tensor | None = None) -> None:
        """Attention only (the cache already holds this step's rows): decodes, then chunks and code steps."""
        nd, nd_tok, n_tok = md.num_decodes, md.num_decode_tokens, md.num_actual_tokens
        if nd:
            torch.ops.abridgekv.decode_attn(q[:nd_tok], kv_cache, md.block_table[:nd], md.seq_lens_dev[:nd],
                                            self.scale, md.max_decode_pages, md.split_pages, out[:nd_tok],
                                            None if lse is None else lse[:nd_tok], md.workspace)
        if nd < md.num_reqs and n_tok > nd_tok:
            qsl = md.query_start_loc[nd:] - nd_tok
            sl = md.seq_lens[nd:]
            qlen = np.diff(qsl)
            lim = md.code_key_limit[nd:]
            code = lim != NOT_CODE
            ex = None if md.code_excluded is None else [tuple(e) if e[1] > e[0] else None
                                                         for e in md.code_excluded[nd:]]
            causal = md.causal & ~code
            if md.code_causal is not None:
                causal = causal | (code & md.code_causal[nd:])
            ops.paged_prefill_attention(q[nd_tok:n_tok], kv_cache, md.block_table[nd:], qsl, sl - qlen,
                                        np.where(code, lim, sl), causal, self.scale,
                                        out=out[nd_tok:n_tok], lse=None if lse is None else lse[nd_tok:n_tok],
                                        excluded=ex)


class AbridgeAttentionBackend:
    """Static description of the backend (the vLLM ``AttentionBackend`` surface the path uses)."""

    @staticmethod
    def get_name() -> str:
        return "ABRIDGEKV_HIP"

    @staticmethod
    def get_impl_cls():
        return AbridgeAttentionImpl

    @staticmethod
    def get_builder_cls():
        return AbridgeMetadataBuilder

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int = ops.PAGE, num_kv_heads: int = ops.HEADS_KV,
                           head_size: int = ops.HEAD_DIM) -> tuple[int, ...]:
        """[num_blocks, 2, block_size, num_kv_heads, head_size] (NHD), the layout the worker allocates once per
        shared layer tensor (gpu_model_runner.py:1215-1217)."""
        if (block_size, num_kv_heads, head_size) != (ops.PAGE, ops.HEADS_KV, ops.HEAD_DIM):
            raise NotImplementedError(f"kernels are built for page {ops.PAGE}, {ops.HEADS_KV} KV heads, "
                                      f"head size {ops.HEAD_DIM}")
        return ops.kv_cache_shape(num_blocks)

    @staticmethod
    def get_supported_head_sizes() -> list[int]:
        return [ops.HEAD_DIM]

    @staticmethod
    def get_supported_kernel_block_sizes() -> list[int]:
        return [ops.PAGE]


def attach(layer, impl: AbridgeAttentionImpl | None = None) -> None:
    """Route a layer's attention through this backend via :func:`maybe_override_attention`."""
    layer._abridgekv_impl = impl if impl is not None else AbridgeAttentionImpl()


def maybe_override_attention(layer: object, query: torch.Tensor, kv_cache: torch.Tensor, attn_metadata: object,
                             output: torch.Tensor) -> None:
    """Overlay hook (compresslm_packed_kv.py:744-761): when ``layer`` carries this backend and the metadata is ours,
    recompute the layer's attention in place into ``output``; otherwise do nothing. Expects the step's K/V rows
    already in ``kv_cache`` (the stock path appends them before the hook runs)."""
    impl = getattr(layer, "_abridgekv_impl", None)
    if impl is None or not isinstance(attn_metadata, AbridgeAttentionMetadata):
        return
    T = query.shape[0]
    impl.attend(query.view(T, impl.num_heads, impl.head_size), kv_cache, attn_metadata,
                output.view(T, impl.num_heads, impl.head_size))
