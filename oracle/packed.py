"""Per-head packed code pages (oracle; test infrastructure only).

Restates the reference's packed KV sidecar (third_party/vllm_overlay/vllm/v1/worker/compresslm_packed_kv.py) in
numpy: the page layout of PackedKVLayout.pack_layer / unpack_layer (:112-155), the capture of a closed block's code
rows (:259-284 with _gather_cache_span :159-183), and the per-head attention of override_attention's reference loop
(:422-484: keys = the head's rows of every packed page, in page order, then the request's paged rows; causal chunks
hide paged rows past each query's position, a code step hides paged rows at or past prefix_len + q_h), in float64.

Pinning:
* ``pack`` / ``unpack``  -- a hand-worked page of a 2-head layout, and unpack(pack(x)) == x on every kept row.
* ``packed_attention_fp64`` -- with equal quotas q in every head it must equal the plain paged attention
  (oracle.decode.decode_fp64 / oracle.masks.masked_paged_attention_fp64, pinned by closed forms) over the rows
  [q code rows of every captured block | paged rows]; each KV head's output depends only on its own quota (the
  output of head h under a mixed schedule equals the output under the uniform schedule q_h); with no captured
  block a code step equals the code-step mask of oracle.masks, also with an excluded range (the block's static tail,
  :725-729).
"""
from __future__ import annotations

import numpy as np

from .decode import paged_rows


def offsets(quota_row):
    return np.concatenate([[0], np.cumsum(np.asarray(quota_row, dtype=np.int64))])


def pack(quota_row, dense):
    """[2, K_max, Hkv, D] -> [2, sum q_h, D]: head h's first q_h rows, heads in order (pack_layer :112-128)."""
    return np.concatenate([dense[:, :q, h, :] for h, q in enumerate(quota_row)], axis=1)


def unpack(quota_row, k_max, packed, fill=0.0):
    """[2, sum q_h, D] -> [2, K_max, Hkv, D], rows past a head's quota = fill (unpack_layer :130-155)."""
    off = offsets(quota_row)
    dense = np.full((2, k_max, len(quota_row), packed.shape[-1]), fill, dtype=packed.dtype)
    for h, q in enumerate(quota_row):
        dense[:, :q, h, :] = packed[:, off[h]: off[h + 1], :]
    return dense


def capture(kv_cache, block_table, start, k_max, quota_row):
    """The packed page of the k_max code rows at physical [start, start + k_max) of one layer (capture :259-284)."""
    pos = np.arange(start, start + k_max)
    pages = np.asarray(block_table, dtype=np.int64)[pos // kv_cache.shape[2]]
    dense = np.stack([kv_cache[pages, 0, pos % kv_cache.shape[2]], kv_cache[pages, 1, pos % kv_cache.shape[2]]])
    return pack(quota_row, dense)


def packed_attention_fp64(q_rows, pages, quota_row, kv_cache, block_table, seq_len, query_len, causal, k_max, scale,
                          excluded=None):
    """One request's attention with side rows (the per-head loop of override_attention, :422-484).

    q_rows [query_len, Hq, D]; pages: the request's packed pages [2, sum q, D] in capture order; the queries are the
    last query_len of the seq_len paged rows; ``excluded``: physical paged rows [start, end) a code step hides (its
    block's static tail, :725-729). Returns (out [query_len, Hq, D], lse [query_len, Hq]) in float64.
    """
    q_rows = np.asarray(q_rows, dtype=np.float64)
    mk, mv = paged_rows(kv_cache, block_table, seq_len)
    Hq, Hkv = q_rows.shape[1], mk.shape[1]
    g = Hq // Hkv
    off = offsets(quota_row)
    prefix = seq_len - query_len
    out = np.zeros(q_rows.shape, dtype=np.float64)
    lse = np.full(q_rows.shape[:2], -np.inf)
    for h in range(Hkv):
        sk = [np.asarray(p[0, off[h]: off[h + 1]], dtype=np.float64) for p in pages]
        sv = [np.asarray(p[1, off[h]: off[h + 1]], dtype=np.float64) for p in pages]
        side = sum(x.shape[0] for x in sk)
        key = np.concatenate(sk + [mk[:, h].astype(np.float64)]) if pages else mk[:, h].astype(np.float64)
        val = np.concatenate(sv + [mv[:, h].astype(np.float64)]) if pages else mv[:, h].astype(np.float64)
        hidden = np.zeros((query_len, key.shape[0]), dtype=bool)
        main_pos = np.arange(seq_len)
        if causal and query_len > 1:
            hidden[:, side:] = main_pos[None, :] >= (prefix + np.arange(1, query_len + 1))[:, None]
        elif not causal:
            if query_len != k_max:
                raise RuntimeError("noncausal step must contain exactly k_max code queries")
            hidden[:, side:] = (main_pos >= prefix + quota_row[h])[None, :]
            if excluded is not None:
                hidden[:, side + excluded[0]: side + excluded[1]] = True
        for gi in range(g):
            hq = h * g + gi
            s = scale * q_rows[:, hq] @ key.T
            s[hidden] = -np.inf
            m = s.max(axis=1, keepdims=True)
            ok = np.isfinite(m[:, 0])
            w = np.where(ok[:, None], np.exp(s - np.where(ok[:, None], m, 0.0)), 0.0)
            l = w.sum(axis=1)
            out[:, hq] = np.where(ok[:, None], (w @ val) / np.where(l > 0, l, 1.0)[:, None], 0.0)
            lse[:, hq] = np.where(ok, m[:, 0] + np.log(np.where(l > 0, l, 1.0)), -np.inf)
    return out, lse
