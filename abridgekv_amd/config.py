"""Serving configuration of the abridged cache (API-compatible subset of the reference's CompressLMConfig).

Mirrors third_party/vllm_overlay/vllm/config/compresslm.py:9-309, with its defaults (appended code positions, a
replay tail of 16), for the configurations its serving path decodes: one pause pass, raw prompt, ``appended`` or
``bitrev`` code positions; either a replay tail of R = replay_tail rows (appended positions: after its codes a block
runs its last R content tokens again; the next block's content token i expires replay row i; with
code_exclude_replay_tail the codes do not see those content rows) or a retained tail of T = retain_tail_kv original
content rows per block (compresslm.py:22-26): "static" keeps the last T content rows of every block resident for
every later query; the window policies keep the previous block's tail for the next block's content queries only,
"rolling" expiring one row per next-block content token and "sticky" all of it before the next block's codes. The
codes of a block summarize only its first C - T content rows (compresslm.py:192-206, 254-257). Optional per-layer
quotas with physical removal (bitrev positions), or per-head quotas in packed KV pages (packed_kv, packed_kv_k_max,
packed_kv_quotas; validated as at compresslm.py:145-190; packed KV takes no window tail). The raw tail and selective
full-history evaluation are rejected with ValueError instead of being silently ignored.
"""
from __future__ import annotations

import json
from collections.abc import Sequence
from dataclasses import dataclass, field, fields
from pathlib import Path

import numpy as np


def layer_index(layer_name: str) -> int | None:
    """Index n of an attention layer named '...layers.n....' (None when not indexed)."""
    marker = ".layers."
    if marker not in layer_name:
        return None
    head = layer_name.split(marker, 1)[1].split(".", 1)[0]
    return int(head) if head.isdigit() else None


def bitrev_offsets(K: int, span: int) -> np.ndarray:
    """Row k of a K-row code block -> floor(bitreverse_{log2 K}(k) * span / K) (int64)."""
    if K <= 0 or K & (K - 1):
        raise ValueError("num_code_tokens must be a power of two for bitrev positions")
    if span < K:
        raise ValueError(f"bitrev code span {span} < num_code_tokens {K}")
    bits = K.bit_length() - 1
    k = np.arange(K, dtype=np.int64)
    rev = np.zeros_like(k)
    for b in range(bits):
        rev |= ((k >> b) & 1) << (bits - 1 - b)
    return (rev * span) // K


def load_quota_rows(path) -> tuple[tuple[int, ...], ...]:
    """(layer x KV head) quota rows of a schedule file: a 2D array, or an object with 'packed_kv_quotas' / 'quotas'
    (scripts/compresslm_schedules.py:6-13)."""
    payload = json.loads(Path(path).read_text())
    if isinstance(payload, dict):
        payload = payload.get("packed_kv_quotas", payload.get("quotas"))
    if not isinstance(payload, list) or not payload:
        raise ValueError(f"{path}: expected a non-empty 2D quota array or an object with 'quotas'")
    return tuple(tuple(int(v) for v in row) for row in payload)


def load_layer_quotas(path) -> tuple[int, ...]:
    """Per-layer quotas for serving: every layer's row must be uniform across KV heads
    (scripts/compresslm_schedules.py:16-25)."""
    quotas = []
    for layer, row in enumerate(load_quota_rows(path)):
        if len(set(row)) != 1:
            raise ValueError(f"{path}: layer {layer} has per-head quotas {sorted(set(row))}; per-layer serving needs "
                             f"one quota per layer")
        quotas.append(row[0])
    return tuple(quotas)


# the fields scripts/convert_compresslm_checkpoint_to_hf.py:189-206 writes into compresslm_config.json
_EXPORT_FIELDS = ("enable", "block_size", "num_code_tokens", "num_passes", "pause_xattn", "raw_prompt", "raw_tail",
                  "replay_tail", "code_positions", "retain_tail_kv", "retain_tail_policy", "code_exclude_replay_tail",
                  "code_token_format")


@dataclass
class CompressLMConfig:
    enable: bool = False
    block_size: int = 512
    num_code_tokens: int = 128
    replay_tail: int = 16
    retain_tail_kv: int = 0
    retain_tail_policy: str = "rolling"
    code_exclude_replay_tail: bool = False
    raw_prompt: bool = True
    num_passes: int = 1
    pause_xattn: str = "full"
    raw_tail: int = 0
    code_token_format: str = "<|compress_code_{:03d}|>"
    debug: bool = False
    code_positions: str = "appended"
    layer_code_quotas: tuple[int, ...] = ()
    physical_layer_quotas: bool = False
    retain_full_history_layers: tuple[int, ...] = ()
    packed_kv: bool = False
    packed_kv_k_max: int = 2048
    packed_kv_quotas: tuple[tuple[int, ...], ...] = ()

    _code_token_ids: list[int] = field(default_factory=list, repr=False)
    _initialized: bool = field(default=False, repr=False)

    def __post_init__(self) -> None:
        self.layer_code_quotas = tuple(int(q) for q in self.layer_code_quotas)
        self.packed_kv_quotas = tuple(tuple(int(v) for v in row) for row in self.packed_kv_quotas)
        self.retain_full_history_layers = tuple(sorted(set(self.retain_full_history_layers)))
        if self.retain_tail_policy not in ("rolling", "sticky", "static"):
            raise ValueError("retain_tail_policy must be one of: rolling, sticky, static")
        if self.code_positions not in ("appended", "bitrev"):
            raise ValueError("code_positions must be appended or bitrev")
        if not self.enable:
            return
        C, K = self.block_size, self.num_code_tokens
        if C <= 0:
            raise ValueError("block_size must be positive")
        if K <= 0:
            raise ValueError("num_code_tokens must be positive")
        if self.code_positions == "bitrev":
            if (C & (C - 1)) or (K & (K - 1)) or self.replay_tail or self.raw_tail or self.num_passes != 1:
                raise ValueError("code_positions=bitrev needs power-of-two block_size and num_code_tokens, "
                                 "no replay/raw tail and num_passes=1")
        if not 0 <= self.replay_tail <= C:
            raise ValueError("replay_tail must be in [0, block_size]")
        if not 0 <= self.retain_tail_kv < C:
            raise ValueError("retain_tail_kv must be in [0, block_size)")
        if self.retain_tail_policy == "sticky" and not self.retain_tail_kv:
            raise ValueError("retain_tail_policy='sticky' requires retain_tail_kv > 0")
        if sum(bool(v) for v in (self.raw_tail, self.replay_tail, self.retain_tail_kv)) > 1:
            raise ValueError("raw_tail, replay_tail, and retain_tail_kv are mutually exclusive")
        if self.code_exclude_replay_tail and not 0 < self.replay_tail < C:
            raise ValueError("code_exclude_replay_tail requires replay_tail in [1, block_size)")
        if self.code_positions == "bitrev" and C - self.code_excluded_tail < K:
            raise ValueError(f"bitrev code span {C - self.code_excluded_tail} < num_code_tokens {K}")
        if self.num_passes != 1:
            raise ValueError("CompressLM decoding supports num_passes=1 only")
        if self.pause_xattn != "full":
            raise ValueError("CompressLM decoding requires pause_xattn='full'")
        if self.raw_tail:
            raise ValueError("vLLM CompressLM decoding currently supports raw_tail=0 only")
        if not self.raw_prompt:
            raise ValueError("CompressLM decoding requires raw_prompt=True")
        if self.retain_full_history_layers:
            raise ValueError("selective full history is not served")
        for layer, q in enumerate(self.layer_code_quotas):
            if not 0 < q <= K:
                raise ValueError(f"layer_code_quotas[{layer}]={q} must be in [1, {K}]")
        if self.uses_layer_quotas and self.code_positions != "bitrev":
            raise ValueError("layer_code_quotas below num_code_tokens need code_positions=bitrev (nested-prefix code "
                             "layout)")
        if self.packed_kv and any(q < K for q in self.layer_code_quotas):
            raise ValueError("layer_code_quotas and packed KV are mutually exclusive")
        if self.packed_kv:
            if self.retain_tail_kv and self.retain_tail_policy != "static":
                raise ValueError("packed KV supports code/replay checkpoints and the static retained tail, not window "
                                 "(rolling/sticky) or raw tails")
            if self.code_exclude_replay_tail:
                raise ValueError("packed KV does not yet support code_exclude_replay_tail")
            if self.packed_kv_k_max != K:
                raise ValueError("packed_kv_k_max must equal num_code_tokens so the dense code pass computes every "
                                 "schedulable slot")
            for layer, row in enumerate(self.packed_kv_quotas):
                if not row:
                    raise ValueError(f"packed_kv_quotas[{layer}] must not be empty")
                for head, q in enumerate(row):
                    if not 0 < q <= self.packed_kv_k_max:
                        raise ValueError(f"packed_kv_quotas[{layer}][{head}]={q} must be in "
                                         f"[1, {self.packed_kv_k_max}]")
        if self.physical_layer_quotas and not self.layer_code_quotas:
            raise ValueError("physical_layer_quotas needs layer_code_quotas")

    # -- compresslm_config.json ------------------------------------------------------------------------------------
    @classmethod
    def from_metadata(cls, metadata: dict, layer_quotas_path=None, physical_layer_quotas: bool = False,
                      **overrides) -> "CompressLMConfig":
        """Config from an export's compresslm_config.json contents, as the serving entry points build it
        (scripts/bench_decode.py:51-58, scripts/eval_math500_compresslm.py:273-285): provenance keys that are not
        config fields are dropped; ``layer_quotas_path`` adds per-layer quotas from a schedule file; recorded
        ``code_token_ids`` are installed."""
        meta = dict(metadata)
        ids = meta.pop("code_token_ids", None)
        names = {f.name for f in fields(cls)}
        meta = {k: v for k, v in meta.items() if k in names and not k.startswith("_")}
        if layer_quotas_path is not None:
            meta["layer_code_quotas"] = load_layer_quotas(layer_quotas_path)
            meta["physical_layer_quotas"] = bool(physical_layer_quotas)
        meta.update(overrides)
        cfg = cls(**meta)
        if ids is not None and cfg.enable:
            cfg.set_code_token_ids(ids)
        return cfg

    @classmethod
    def from_json(cls, path, **kwargs) -> "CompressLMConfig":
        """Load ``<model_dir>/compresslm_config.json`` (or the file itself)."""
        p = Path(path)
        if p.is_dir():
            p = p / "compresslm_config.json"
        return cls.from_metadata(json.loads(p.read_text()), **kwargs)

    def to_metadata(self) -> dict:
        """The compresslm_config.json contents (scripts/convert_compresslm_checkpoint_to_hf.py:189-206, 244), plus
        the code token ids when they are installed."""
        meta = {name: getattr(self, name) for name in _EXPORT_FIELDS}
        if self._initialized:
            meta["code_token_ids"] = list(self._code_token_ids)
        return meta

    def write_json(self, path) -> Path:
        p = Path(path)
        if p.is_dir():
            p = p / "compresslm_config.json"
        p.write_text(json.dumps(self.to_metadata(), indent=2) + "\n")
        return p

    # -- positions ------------------------------------------------------------------------------------------------
    @property
    def code_excluded_tail(self) -> int:
        """Content rows at the end of each block that the block's own codes never see and do not summarize: the
        replayed rows with code_exclude_replay_tail, else the retained tail, whatever its policy
        (compresslm.py:254-260)."""
        return self.replay_tail if self.code_exclude_replay_tail else self.retain_tail_kv

    def bitrev_code_offsets(self) -> np.ndarray:
        """In-block RoPE offsets of the code rows (config/compresslm.py:192-206)."""
        return bitrev_offsets(self.num_code_tokens, self.block_size - self.code_excluded_tail)

    def bitrev_rope_positions(self, logical) -> np.ndarray:
        """Logical positions (period C+K per block) -> bitrev RoPE positions (config/compresslm.py:208-216)."""
        C, K = self.block_size, self.num_code_tokens
        logical = np.asarray(logical, dtype=np.int64)
        blk, within = logical // (C + K), logical % (C + K)
        offs = self.bitrev_code_offsets()[np.clip(within - C, 0, K - 1)]
        return blk * C + np.where(within >= C, offs, within)

    # -- token ids ------------------------------------------------------------------------------------------------
    def initialize_token_ids(self, tokenizer) -> "CompressLMConfig":
        if self._initialized:
            return self
        if tokenizer is None:
            raise ValueError("CompressLM decoding requires an initialized tokenizer")
        ids = []
        for token in self.code_tokens:
            enc = tokenizer.encode(token, add_special_tokens=False)
            if len(enc) != 1:
                raise ValueError(f"CompressLM code token {token!r} must encode to one ID; got {enc}")
            ids.append(enc[0])
        if len(set(ids)) != len(ids):
            raise ValueError("CompressLM code tokens must have distinct token IDs")
        self._code_token_ids, self._initialized = ids, True
        return self

    def set_code_token_ids(self, ids: Sequence[int]) -> "CompressLMConfig":
        """Install code-token ids directly (tokenizer-free use, tests)."""
        ids = [int(i) for i in ids]
        if len(ids) != self.num_code_tokens or len(set(ids)) != len(ids):
            raise ValueError("need num_code_tokens distinct code token ids")
        self._code_token_ids, self._initialized = ids, True
        return self

    @property
    def code_token_ids(self) -> list[int]:
        if not self._initialized:
            raise RuntimeError("Call initialize_token_ids() before decoding")
        return self._code_token_ids

    @property
    def code_tokens(self) -> list[str]:
        return [self.code_token_format.format(i) for i in range(self.num_code_tokens)]

    # -- quotas ---------------------------------------------------------------------------------------------------
    @property
    def uses_layer_quotas(self) -> bool:
        return any(q < self.num_code_tokens for q in self.layer_code_quotas)

    @property
    def uses_physical_layer_quotas(self) -> bool:
        return bool(self.physical_layer_quotas) and self.uses_layer_quotas

    @property
    def uses_selective_history(self) -> bool:
        return False

    @property
    def uses_packed_kv(self) -> bool:
        return bool(self.packed_kv)

    def packed_layout(self, num_layers: int, num_kv_heads: int = 8):
        """The PackedKVLayout of this config (uniform k_max rows when no schedule is given)."""
        from .packed_kv import PackedKVLayout
        return PackedKVLayout.from_schedule(self.packed_kv_quotas or None, num_layers=num_layers,
                                            num_kv_heads=num_kv_heads, k_max=self.packed_kv_k_max)

    def layer_quota(self, layer: int) -> int:
        if 0 <= layer < len(self.layer_code_quotas):
            return self.layer_code_quotas[layer]
        return self.num_code_tokens

    @property
    def distinct_layer_quotas(self) -> tuple[int, ...]:
        return tuple(sorted(set(self.layer_code_quotas)))

    def kv_group_quotas(self, group_layer_names: Sequence[Sequence[str]]) -> tuple[int, ...]:
        """Quota of every KV-cache group; a group must hold layers of one quota."""
        out = []
        for names in group_layer_names:
            qs = set()
            for name in names:
                idx = layer_index(name)
                if idx is None:
                    raise ValueError(f"physical per-layer quotas need indexed attention layers; got {name!r}")
                qs.add(self.layer_quota(idx))
            if len(qs) != 1:
                raise ValueError(f"KV cache group mixes code quotas {sorted(qs)}: {list(names)}")
            out.append(qs.pop())
        return tuple(out)

    def kv_cache_groups(self, num_layers: int) -> tuple[list[list[int]], list[int]]:
        """(layers per KV-cache group, quota per group) for a model of ``num_layers`` attention layers, grouped as the
        reference's KV-cache config does (kv_cache_utils.py:1001-1052, 1216-1226)."""
        from .workloads import quota_groups

        return quota_groups([self.layer_quota(i) for i in range(num_layers)])
