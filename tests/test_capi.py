"""The C-ABI library loads without a GPU and exports every function declared in include/*.h; the Python binding
table covers the same set."""
import re
import subprocess
from pathlib import Path

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


def test_binding_table_matches_header():
    assert set(_lib.SIGNATURES) == declared_functions()


def test_host_only_entry_points_run_without_gpu():
    lib = _lib.lib()
    assert lib.abkv_decode_workspace_size(256, 24) == 256 * 24 * 32 * 130 * 4
    assert lib.abkv_kv_stage_bytes(6, 100, 2048) == 6 * 100 * 4096
    h = lib.abkv_planner_create(8, 2, 4, None, 0)
    assert h
    assert lib.abkv_planner_num_free(h) == 7
    lib.abkv_planner_destroy(h)
