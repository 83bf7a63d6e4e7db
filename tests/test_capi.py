"""The C-ABI library loads without a GPU and exports every function declared in include/*.h; the Python binding
table covers the same set."""
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from abridgekv_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(abkv_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_declares_functions():
    assert len(declared_functions()) >= 25


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in sorted(declared_functions()):
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (abkv_[a-z0-9_]+)", out))
    assert declared_functions() <= exported
    assert exported <= declared_functions(), f"undeclared exports: {sorted(exported - declared_functions())}"


def test_probe_library_loads_and_exports_only_the_probe():
    """The benchmark's measurement probes live in their own library, outside the C-ABI boundary."""
    import ctypes

    path = _lib.LIB_PATH.parent / "libabridgekv_probes.so"
    ctypes.CDLL(str(path))
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True).stdout
    assert set(re.findall(r" T (abkv_[a-z0-9_]+)", out)) == {"abkv_probe_row_copy"}


def test_binding_table_matches_header():
    assert set(_lib.SIGNATURES) == declared_functions()


def test_host_only_entry_points_run_without_gpu():
    lib = _lib.lib()
    # per (sequence, split, query head): 128 fp16 partial values + an fp32 record (m, l, scale, unused)
    assert lib.abkv_decode_workspace_size(256, 24) == 256 * 24 * 32 * (128 * 2 + 4 * 4)
    assert lib.abkv_kv_stage_bytes(6, 100, 2048) == 6 * 100 * 4096
    h = lib.abkv_planner_create(8, 2, 4, None, 0)
    assert h
    assert lib.abkv_planner_num_free(h) == 7
    lib.abkv_planner_destroy(h)


def test_rope_table_matches_hf_rotary():
    """The fp32 cos/sin table equals HF's default rotary embedding values and is close to the float64 closed form."""
    import math

    import torch
    transformers = pytest.importorskip("transformers")
    from abridgekv_amd import ops

    table = ops.rope_cos_sin_cache(4096, theta=1e6)
    cfg = transformers.Qwen3Config(hidden_size=256, num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                                   rope_parameters={"rope_theta": 1e6, "rope_type": "default"})
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding
    hf = ops.rotary_cos_sin_from_model(Qwen3RotaryEmbedding(cfg), 4096, "cpu")
    assert torch.equal(table, hf)
    pos, i = 1234, 5
    want = math.cos(pos * 1e6 ** (-2 * i / 128))
    assert abs(table[pos, i].item() - want) < 1e-4


@pytest.mark.parametrize("C,K", [(64, 16), (48, 16), (512, 256)])
def test_rope_bound_is_the_running_maximum_of_the_bitrev_positions(C, K):
    """ops.rope_bound(p) = max RoPE position over logical positions 0..p (brute force over the oracle's layout)."""
    from abridgekv_amd import ops
    from oracle import layout as ol
    logical = np.arange(6 * (C + K))
    running = np.maximum.accumulate(ol.bitrev_rope_positions(logical, C, K))
    got = np.array([ops.rope_bound(int(p), C, K) for p in logical])
    assert np.array_equal(got, running)
    assert ops.rope_bound(1234) == 1234
