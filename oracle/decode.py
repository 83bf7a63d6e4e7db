"""Decode attention over the abridged paged cache (oracle; test infrastructure only).

Pinning:
* ``paged_rows``         -- slot = table[pos // 16] * 16 + pos % 16; pinned by a brute-force page walk in
                            tests/test_oracle_decode.py.
* ``decode_fp64``        -- pinned by special cases with closed forms: one row (output == v, lse == s), identical
                            rows (output == v, lse == s + log n), two rows (logistic weights), permutation
                            invariance of rows, and agreement with scipy.special.logsumexp / softmax.
* ``decode_ref_torch``   -- the reference's own arithmetic on CPU torch; pinned against decode_fp64 within the bf16
                            bound (it is a measurement baseline, not a parity target).
* ``request_ref_torch``  -- the reference's per-request multi-query arithmetic (code step / prompt chunk) on CPU
                            torch; pinned against decode_fp64 row by row within the bf16 bound, with a planted value
                            row just past each query's visible range that would break the bound if it were read.
"""
from __future__ import annotations

import numpy as np

from .layout import PAGE


def paged_rows(kv_cache: np.ndarray, block_table: np.ndarray, seq_len: int, page: int = PAGE):
    """Gather the first ``seq_len`` physical rows of one sequence from a [P, 2, page, Hkv, D] cache.

    Restates the slot map of third_party/vllm_overlay/vllm/v1/worker/block_table.py:186-197 (non-CP branch) and
    the cache layout of gpu_model_runner.py:1215-1217 ([num_blocks, 2, block_size, num_kv_heads, head_size]).
    Returns (K [n, Hkv, D], V [n, Hkv, D]).
    """
    pos = np.arange(seq_len, dtype=np.int64)
    pages = np.asarray(block_table, dtype=np.int64)[pos // page]
    offs = pos % page
    return kv_cache[pages, 0, offs], kv_cache[pages, 1, offs]


def decode_fp64(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float):
    """softmax(scale * q_h . K^T) V for every query head h, GQA (query head h reads KV head h // (Hq / Hkv)).

    Restates the attention math of abridgekv/gen_compress.py:359-360, :555 and
    third_party/vllm_overlay/vllm/v1/worker/compresslm_packed_kv.py:608-613 over all resident rows (decode under
    physical quotas needs no mask: gpu_model_runner.py:2042-2050), in float64.
    q: [Hq, D]; k, v: [n, Hkv, D]. Returns (out [Hq, D] float64, lse [Hq] float64, natural log).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    Hq, D = q.shape
    n, Hkv, _ = k.shape
    if n == 0:
        return np.zeros((Hq, D)), np.full(Hq, -np.inf)
    g = Hq // Hkv
    kh = np.repeat(k.transpose(1, 0, 2), g, axis=0)          # [Hq, n, D]
    vh = np.repeat(v.transpose(1, 0, 2), g, axis=0)
    s = np.einsum("hd,hnd->hn", q, kh) * scale
    m = s.max(axis=1, keepdims=True)
    e = np.exp(s - m)
    z = e.sum(axis=1, keepdims=True)
    out = np.einsum("hn,hnd->hd", e / z, vh)
    lse = (m + np.log(z))[:, 0]
    return out, lse


def decode_paged_fp64(q, kv_cache, block_tables, seq_lens, scale, page: int = PAGE):
    """Batched fp64 decode over a paged cache. q [B, Hq, D] -> (out [B, Hq, D], lse [B, Hq])."""
    B, Hq, D = q.shape
    out = np.zeros((B, Hq, D))
    lse = np.zeros((B, Hq))
    for b in range(B):
        k, v = paged_rows(kv_cache, block_tables[b], int(seq_lens[b]), page)
        out[b], lse[b] = decode_fp64(q[b], k, v, scale)
    return out, lse


def decode_ref_torch(q, kv_cache, block_table, seq_lens, scale, page: int = PAGE):
    """The reference's decode arithmetic on CPU torch, used as the timed CPU baseline.

    Gather through the block table, then scores in the cache dtype, fp32 softmax, probabilities cast back to the
    cache dtype, probabilities x V: third_party/vllm_overlay/vllm/v1/worker/compresslm_packed_kv.py:564-616
    (_attend_decode_batched: gather, einsum, masked_fill, softmax(dtype=float32).to(q.dtype), einsum) and
    abridgekv/gen_compress.py:359-360, :555. Ragged batches are padded to the longest sequence and masked,
    exactly as the reference's batched index does (``hidden`` columns -> -inf).
    q: [B, Hq, D] torch tensor; kv_cache: [P, 2, page, Hkv, D]; block_table [B, W] int; seq_lens [B] int.
    Returns out [B, Hq, D] in q's dtype.
    """
    import torch

    B, Hq, D = q.shape
    Hkv = kv_cache.shape[3]
    g = Hq // Hkv
    S = int(seq_lens.max())
    pos = torch.arange(S)
    hidden = pos.unsqueeze(0) >= seq_lens.view(-1, 1).to(torch.long)                  # [B, S]
    pidx = (pos // page).clamp(max=block_table.shape[1] - 1)
    blocks = block_table.to(torch.long)[:, pidx]                                      # [B, S]
    offs = (pos % page).unsqueeze(0).expand(B, S)
    main = kv_cache[blocks, :, offs]                                                  # [B, S, 2, Hkv, D]
    key = main[:, :, 0].permute(0, 2, 1, 3)                                           # [B, Hkv, S, D]
    value = main[:, :, 1].permute(0, 2, 1, 3)
    qq = q.reshape(B, Hkv, g, D)
    scores = torch.einsum("rhgd,rhtd->rhgt", qq, key) * scale
    scores.masked_fill_(hidden.view(B, 1, 1, S), -torch.inf)
    weights = torch.softmax(scores, dim=-1, dtype=torch.float32).to(q.dtype)
    attended = torch.einsum("rhgt,rhtd->rhgd", weights, value)
    return attended.reshape(B, Hq, D)


def request_ref_torch(q, key, value, scale, limit: int, causal: bool = False, prefix_len: int = 0):
    """The reference's multi-query attention of one request on CPU torch, used as the timed CPU baseline of the code
    step: third_party/vllm_overlay/vllm/v1/worker/compresslm_packed_kv.py:648-745 (_attend_request_vectorized: one
    einsum over all KV heads, hidden keys -> -inf, softmax(dtype=float32).to(q.dtype), einsum), main rows only.

    q [n, Hq, D]; key / value [Hkv, S, D] (the request's physical rows); query i sees keys < limit, and when causal
    also keys <= prefix_len + i (the code step is non-causal with limit = code start + quota). Returns [n, Hq, D].
    """
    import torch

    n, Hq, D = q.shape
    Hkv, S = key.shape[0], key.shape[1]
    g = Hq // Hkv
    qq = q.reshape(n, Hkv, g, D)
    scores = torch.einsum("qhgd,htd->qhgt", qq, key) * scale
    pos = torch.arange(S)
    hidden = (pos >= limit).unsqueeze(0).expand(n, S)
    if causal:
        hidden = hidden | (pos.unsqueeze(0) >= (prefix_len + torch.arange(1, n + 1)).unsqueeze(1))
    scores.masked_fill_(hidden.view(n, 1, 1, S), -torch.inf)
    weights = torch.softmax(scores, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.einsum("qhgt,htd->qhgd", weights, value).reshape(n, Hq, D)
