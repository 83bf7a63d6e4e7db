"""Token/row layout of the abridged cache (oracle; test infrastructure only).

Pinning:
* ``bitrev_code_offsets``  -- pinned by closed forms (K=256 -> 2*bitrev8(k); prefix-K independence; distinctness;
  max < span) in tests/test_oracle_layout.py, which are the reference's own test invariants
  (scripts/test_compresslm_vllm_state.py:349-353).
* ``bitrev_rope_positions`` -- pinned against brute-force enumeration of the [C content | K codes] block stream.
* ``rope_neox``            -- pinned against an explicit complex-rotation formula and norm preservation.
* ``quota_groups``         -- pinned against the grouping the reference's own test asserts
  (scripts/test_compresslm_physical_quotas.py:141-167: 6 groups of 6, quotas [64,64,128,128,128,256]).
* ``rows_per_layer``       -- pinned against a brute-force replay of the compaction trace (oracle.trace).
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

BLOCK_C = 512          # content tokens per block (README.md:8-19)
CODES_K_MAX = 256      # pause (code) rows computed per block in the per-layer arm (launch/train.sh:19)
PAGE = 16              # tokens per KV page (vLLM block size used by the reference serving runs)
ROPE_THETA = 1.0e6     # Qwen3 rope theta

# Per-layer code quotas of the paper's per-layer arm: results/schedules/sched_trunc_perlayer_mean128.json
# (8 heads per layer, all heads of a layer share the quota; layer quota = row[0]).
PERLAYER_MEAN128_QUOTAS = (
    256, 64, 64, 64, 64, 64, 64, 128, 64, 128, 64, 128, 128, 128, 128, 256, 128, 128,
    256, 128, 256, 256, 128, 128, 256, 128, 128, 128, 128, 128, 64, 64, 64, 128, 128, 64,
)


def load_schedule_quotas(path: str | Path) -> tuple[int, ...]:
    """Layer quotas from a per-(layer, head) schedule JSON (results/schedules/*.json format: a list of per-layer
    lists of per-KV-head quotas). Serving with physical quotas needs one quota per layer
    (config/compresslm.py:132-153), so every head of a layer must agree."""
    rows = json.loads(Path(path).read_text())
    out = []
    for li, row in enumerate(rows):
        if len(set(row)) != 1:
            raise ValueError(f"layer {li} mixes head quotas {sorted(set(row))}")
        out.append(int(row[0]))
    return tuple(out)


def bitrev_code_offsets(K: int, C: int, span: int | None = None) -> np.ndarray:
    """In-block RoPE offsets of the K code rows: row k -> floor(bitreverse_{log2 K}(k) * span / K).

    Restates third_party/vllm_overlay/vllm/config/compresslm.py:192-206 and abridgekv/compress_forward.py:46-60.
    """
    span = C if span is None else int(span)
    if K <= 0 or K & (K - 1):
        raise ValueError("K must be a power of two")
    if span < K:
        raise ValueError(f"bitrev code span {span} < K={K}: offsets would collide")
    bits = K.bit_length() - 1
    k = np.arange(K, dtype=np.int64)
    rev = np.zeros_like(k)
    for b in range(bits):
        rev |= ((k >> b) & 1) << (bits - 1 - b)
    return (rev * span) // K


def bitrev_rope_positions(logical, C: int, K: int, span: int | None = None) -> np.ndarray:
    """Logical serving positions (period C+K per block: C content then K codes) -> bitrev RoPE positions.

    Restates third_party/vllm_overlay/vllm/config/compresslm.py:208-216.
    """
    logical = np.asarray(logical, dtype=np.int64)
    blk, within = logical // (C + K), logical % (C + K)
    code = within >= C
    offs = bitrev_code_offsets(K, C, span)[np.clip(within - C, 0, K - 1)]
    return blk * C + np.where(code, offs, within)


def training_rope_positions(N: int, C: int, K: int, K_act: int | None = None, span: int | None = None) -> np.ndarray:
    """RoPE positions of the teacher-forced layout [C content | K_act codes] x N (bitrev code positions).

    Restates the bitrev branch of abridgekv/compress_forward.py:1044-1071 (_rope_position_ids, no copy region).
    """
    K_act = K if K_act is None else K_act
    per = C + K_act
    idx = np.arange(N * per, dtype=np.int64)
    within, blk = idx % per, idx // per
    pos = blk * C + within
    is_code = within >= C
    pos[is_code] = blk[is_code] * C + bitrev_code_offsets(K, C, span)[within[is_code] - C]
    return pos


def rope_inv_freq(head_dim: int, theta: float = ROPE_THETA) -> np.ndarray:
    """Default HF rotary inverse frequencies: theta^(-2i/d), i < d/2 (the Qwen3 rotary embedding)."""
    return 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim))


def rope_neox(x: np.ndarray, positions: np.ndarray, theta: float = ROPE_THETA) -> np.ndarray:
    """Rotate-half (NeoX) RoPE in float64: x * cos + rotate_half(x) * sin with cos/sin = cat(f, f).

    Restates abridgekv/gen_compress.py:34-41 (rotate_half / apply_rope) with the HF default frequencies.
    ``x``: [..., S, H, D]; ``positions``: [S].
    """
    D = x.shape[-1]
    f = np.outer(np.asarray(positions, dtype=np.float64), rope_inv_freq(D, theta))   # [S, D/2]
    emb = np.concatenate([f, f], axis=-1)                                             # [S, D]
    cos, sin = np.cos(emb)[:, None, :], np.sin(emb)[:, None, :]                       # [S, 1, D]
    x = np.asarray(x, dtype=np.float64)
    half = D // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return x * cos + rot * sin


def quota_groups(layer_quotas) -> tuple[list[list[int]], list[int]]:
    """KV-cache groups of a per-layer quota model: (layers per group, quota per group).

    Restates third_party/vllm_overlay/vllm/v1/core/kv_cache_utils.py:1216-1226 (quota specs differ -> hybrid-style
    grouping) and :1001-1052 (_get_kv_cache_groups_uniform_page_size): layers are bucketed by spec in first-appearance
    order; group_size = min bucket size (or the max if max < 1.25*min); bucket i splits into layers[i::n].
    """
    buckets: dict[int, list[int]] = {}
    for layer, q in enumerate(layer_quotas):
        buckets.setdefault(int(q), []).append(layer)
    sizes = [len(v) for v in buckets.values()]
    group_size = min(sizes)
    if max(sizes) < min(sizes) * 1.25:
        group_size = max(sizes)
    groups, quotas = [], []
    for q, layers in buckets.items():
        n = -(-len(layers) // group_size)
        for i in range(n):
            groups.append(layers[i::n])
            quotas.append(q)
    return groups, quotas


def closed_blocks(T: int, C: int = BLOCK_C) -> int:
    """Blocks already compacted when the query is content token T-1 (its own block is still open)."""
    return (T - 1) // C if T > 0 else 0


def rows_per_layer(T: int, P: int, q: int, C: int = BLOCK_C) -> int:
    """Resident rows of one layer (quota q) at a decode query that is content token T-1 (T counts the query).

    Prompt rows are never removed (processor.py:480-483), every closed block keeps q code rows
    (processor.py:537-556), the open block keeps all its rows.
    """
    nb = closed_blocks(T, C)
    return min(P, nb * C) + nb * q + (T - nb * C)
