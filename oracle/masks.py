"""Serving-side custom masks of a CompressLM step (oracle; test infrastructure only).

Restates third_party/vllm_overlay/vllm/v1/worker/compresslm_masks.py:165-239 (build_layer_quota_masks) as plain
numpy loops: per request a (query_len x seq_len) matrix, rows at physical positions seq_len - query_len + i, the
step's ordinary visibility (causal, or everything for the non-causal code step) minus an excluded range, minus
columns [start + q, end) of every code span when q < K. The flat result is the row-major concatenation FlashInfer
consumes (compresslm_masks.py:237-238: ``mask[valid]``).

Also the dense-mask attention over paged rows used to check the attention backend's code-step limits.

Pinning: tests/test_backend.py checks the causal case against np.tril, the code-step case against the hand-derived
"keys < code_start + q" prefix for every quota, the exclusion-range and multi-span cases by brute force over
columns, and masked_paged_attention_fp64 against decode_fp64 when the mask is a prefix.
"""
from __future__ import annotations

import numpy as np

from . import decode as od


def request_mask(query_len, seq_len, spans, excluded, quota, num_code_tokens, causal):
    """One request's bool [query_len, seq_len] (compresslm_masks.py:189-235, one row of ``requests``)."""
    if query_len <= 0 or query_len > seq_len:
        raise ValueError("invalid query_len/seq_len in layer-quota mask build")
    m = np.zeros((query_len, seq_len), dtype=bool)
    for i in range(query_len):
        pos = seq_len - query_len + i
        for c in range(seq_len):
            ok = c <= pos if causal else True
            if excluded is not None and excluded[0] <= c < excluded[1]:
                ok = False
            if quota < num_code_tokens:
                for start, end in spans:
                    if start + quota <= c < end:
                        ok = False
            m[i, c] = ok
    return m


def layer_quota_mask(requests, quota, num_code_tokens, causal):
    """Flat mask of one quota over ``requests`` = [(query_len, seq_len, code_spans, excluded_range)]."""
    if not requests:
        return np.zeros(0, dtype=bool)
    return np.concatenate([request_mask(ql, sl, spans, ex, quota, num_code_tokens, causal).reshape(-1)
                           for ql, sl, spans, ex in requests])


def masked_paged_attention_fp64(q_rows, cache, table, seq_len, mask_rows, scale):
    """fp64 attention of q_rows [n, 32, 128] over the request's first seq_len physical rows, row i seeing the keys
    where mask_rows[i] is true. Rows with no visible key give zeros and LSE -inf."""
    k, v = od.paged_rows(cache, table, seq_len)
    out = np.zeros((len(q_rows), q_rows.shape[1], q_rows.shape[2]))
    lse = np.full((len(q_rows), q_rows.shape[1]), -np.inf)
    for i in range(len(q_rows)):
        idx = np.flatnonzero(mask_rows[i])
        if idx.size:
            out[i], lse[i] = od.decode_fp64(q_rows[i], k[idx], v[idx], scale)
    return out, lse
