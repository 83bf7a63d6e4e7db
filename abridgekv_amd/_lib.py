"""ctypes binding of libabridgekv_amd.so (the C-ABI declared in include/abridgekv_amd.h).

The library is loaded from the package directory only. A missing library is an error: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libabridgekv_amd.so"

_i32p = C.POINTER(C.c_int32)
_i64p = C.POINTER(C.c_int64)
_vp = C.c_void_p

# name -> (restype, argtypes). Keep in the order of include/abridgekv_amd.h.
SIGNATURES = {
    "abkv_decode_workspace_size": (C.c_size_t, [C.c_int, C.c_int]),
    "abkv_decode_attn": (C.c_int, [_vp, C.c_long, C.c_long, _vp, C.c_int, _vp, C.c_long, _vp, C.c_int, C.c_int, C.c_int,
                                   C.c_float, _vp, C.c_long, C.c_long, _vp, _vp, C.c_size_t, _vp]),
    "abkv_decode_attn_noalloc": (C.c_int, [_vp, C.c_long, C.c_long, _vp, C.c_int, _vp, C.c_long, _vp, C.c_int,
                                           C.c_int, C.c_int, C.c_float, _vp, C.c_long, C.c_long, _vp, _vp]),
    "abkv_kv_move_segments": (C.c_int, [C.POINTER(_vp), C.c_int, C.c_int, C.c_int, C.c_long, C.c_long, C.c_int,
                                        _vp, _vp, C.c_int, _vp]),
    "abkv_kv_move_mixed": (C.c_int, [C.POINTER(_vp), C.c_int, C.c_int, C.c_int, C.c_long, C.c_long, C.c_int,
                                     _vp, _vp, C.c_int, _vp, C.c_int, _vp]),
    "abkv_kv_stage_bytes": (C.c_size_t, [C.c_int, C.c_int, C.c_int]),
    "abkv_kv_copy_staged": (C.c_int, [C.POINTER(_vp), C.c_int, C.c_int, C.c_int, C.c_long, C.c_long, C.c_int, _vp,
                                      C.c_int, _vp, C.c_size_t, _vp]),
    "abkv_kv_append": (C.c_int, [_vp, C.c_long, _vp, C.c_long, _vp, C.c_int, _vp, C.c_int, C.c_long, C.c_long,
                                 C.c_int, C.c_int, _vp]),
    "abkv_rope_kv_append": (C.c_int, [_vp, C.c_long, C.c_long, _vp, C.c_long, _vp, C.c_long, _vp, C.c_int, C.c_int,
                                      C.c_int, C.c_int, _vp, C.c_long, _vp, _vp, C.c_int, _vp]),
    "abkv_decode_attn_f32": (C.c_int, [_vp, C.c_long, C.c_long, _vp, C.c_int, _vp, C.c_long, _vp, C.c_int, C.c_int,
                                       C.c_float, _vp, C.c_long, C.c_long, _vp, _vp]),
    "abkv_paged_prefill_attn_f32": (C.c_int, [_vp, C.c_long, C.c_long, _vp, C.c_int, _vp, C.c_long, C.c_int, _vp,
                                              _vp, _vp, _vp, _vp, C.c_int, _vp, C.c_int, C.c_float, _vp, C.c_long,
                                              C.c_long, _vp, _vp]),
    "abkv_prefill_masked_attn_f32": (C.c_int, [_vp, C.c_long, C.c_long, C.c_long, _vp, C.c_long, C.c_long, C.c_long,
                                               _vp, C.c_long, C.c_long, C.c_long, C.c_int, C.c_int, C.c_int, C.c_int,
                                               C.c_int, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                               C.c_int, C.c_int, C.c_float, _vp, C.c_long, C.c_long, C.c_long, _vp,
                                               _vp]),
    "abkv_slot_mapping": (C.c_int, [_vp, _vp, C.c_int, _vp, C.c_int, C.c_long, C.c_int, _vp, _vp, _vp]),
    "abkv_prefill_masked_attn": (C.c_int, [_vp, C.c_long, C.c_long, C.c_long, _vp, C.c_long, C.c_long, C.c_long,
                                           _vp, C.c_long, C.c_long, C.c_long, C.c_int, C.c_int, C.c_int, C.c_int,
                                           C.c_int, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                           C.c_int, C.c_float, _vp, C.c_long, C.c_long, C.c_long, _vp, _vp]),
    "abkv_prefill_masked_bwd_workspace_size": (C.c_size_t, [C.c_int, C.c_int]),
    "abkv_prefill_masked_attn_bwd": (C.c_int, [_vp, C.c_long, C.c_long, C.c_long] * 5
                                     + [_vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp, C.c_int,
                                        C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
                                     + [_vp, C.c_long, C.c_long, C.c_long] * 3 + [_vp, C.c_size_t, _vp]),
    "abkv_paged_prefill_workspace_size": (C.c_size_t, [C.c_int, C.c_int]),
    "abkv_paged_prefill_attn": (C.c_int, [_vp, C.c_long, C.c_long, _vp, C.c_int, _vp, C.c_long, C.c_int, _vp, _vp,
                                          _vp, _vp, _vp, _vp, C.c_int, _vp, C.c_int, C.c_float, _vp, C.c_long,
                                          C.c_long, _vp, C.c_int, C.c_int, C.c_int, _vp, C.c_size_t, _vp]),
    "abkv_packed_capture": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, _vp, C.c_long, C.c_int, _vp,
                                      _vp, C.c_int, _vp]),
    "abkv_decode_side_split_rows": (C.c_int, [C.c_int]),
    "abkv_decode_packed_workspace_size": (C.c_size_t, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "abkv_decode_attn_packed": (C.c_int, [_vp, C.c_long, C.c_long, _vp, C.c_int, _vp, C.c_long, _vp, C.c_int, C.c_int,
                                          C.c_int, _vp, C.c_int, C.c_int, _i32p, _vp, C.c_long, _vp, C.c_int, C.c_int,
                                          C.c_float, _vp, C.c_long, C.c_long, _vp, _vp, C.c_size_t, _vp]),
    "abkv_paged_prefill_attn_packed": (C.c_int, [_vp, C.c_long, C.c_long, _vp, C.c_int, _vp, C.c_long, C.c_int, _vp,
                                                 _vp, _vp, _vp, _vp, _vp, C.c_int, _vp, C.c_int, _vp, _vp, C.c_int,
                                                 C.c_int, _i32p, _vp, C.c_long, _vp, C.c_int, C.c_float, _vp,
                                                 C.c_long, C.c_long, _vp, C.c_int, C.c_int, C.c_int, C.c_int,
                                                 C.c_int, _vp, C.c_size_t, _vp]),
    "abkv_planner_create": (_vp, [C.c_int, C.c_int, C.c_int, _i32p, C.c_int64]),
    "abkv_planner_destroy": (None, [_vp]),
    "abkv_planner_set_op_rows": (C.c_int, [_vp, C.c_int]),
    "abkv_planner_last_error": (C.c_char_p, [_vp]),
    "abkv_planner_add_request": (C.c_int, [_vp, C.c_int64]),
    "abkv_planner_free_request": (C.c_int, [_vp, C.c_int64]),
    "abkv_planner_set_num_computed": (C.c_int, [_vp, C.c_int64, C.c_int64]),
    "abkv_planner_get_num_computed": (C.c_int64, [_vp, C.c_int64]),
    "abkv_planner_allocate_slots": (C.c_int, [_vp, C.c_int64, C.c_int64]),
    "abkv_planner_mask_token_span": (C.c_int, [_vp, C.c_int64, C.c_int64, C.c_int64, _i32p, C.c_int, _i64p,
                                               _i64p]),
    "abkv_planner_pending_sizes": (C.c_int, [_vp, _i64p, _i64p, _i64p]),
    "abkv_planner_take_step_outputs": (C.c_int, [_vp, _i64p, C.c_int64, _i64p, _i64p, C.c_int64, _i64p, _i64p,
                                                 C.c_int64, _i64p]),
    "abkv_moves_pack": (C.c_int64, [_i64p, C.c_int64, C.c_int, _i32p, C.c_int64, _i64p]),
    "abkv_planner_take_moves_packed": (C.c_int64, [_vp, _i64p, C.c_int64, _i64p, _i32p, C.c_int64, _i64p]),
    "abkv_planner_pending_run_sizes": (C.c_int, [_vp, _i64p, _i64p]),
    "abkv_planner_take_move_runs": (C.c_int, [_vp, _i64p, C.c_int64, _i64p, _i32p, C.c_int64, _i32p, C.c_int64, _i32p,
                                              _i64p, _i64p]),
    "abkv_moves_expand": (C.c_int, [_vp, C.c_int, _vp, C.c_long, _vp, C.c_int, C.c_int, _vp, C.c_long, _vp]),
    "abkv_planner_num_free": (C.c_int64, [_vp]),
    "abkv_planner_free_queue": (C.c_int64, [_vp, _i32p, C.c_int64]),
    "abkv_planner_block_ids": (C.c_int64, [_vp, C.c_int64, C.c_int, _i32p, C.c_int64]),
    "abkv_planner_fill_block_table": (C.c_int, [_vp, _i64p, C.c_int, C.c_int, _i32p, C.c_int64, C.c_int32]),
    "abkv_planner_compacted": (C.c_int64, [_vp, C.c_int64, C.c_int]),
    "abkv_planner_spans": (C.c_int64, [_vp, C.c_int64, C.c_int, _i64p, C.c_int64]),
    "abkv_planner_logical_to_physical": (C.c_int64, [_vp, C.c_int64, C.c_int, C.c_int64]),
    "abkv_planner_physical_to_logical": (C.c_int64, [_vp, C.c_int64, C.c_int, C.c_int64]),
    "abkv_planner_is_token_active": (C.c_int, [_vp, C.c_int64, C.c_int, C.c_int64]),
    "abkv_planner_apply_events": (C.c_int64, [_vp, _i64p, C.c_int64]),
}

_LIB = None


def lib():
    """Load (once) and return the bound library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"abridgekv_amd native library missing at {LIB_PATH}; build it with "
                               "`python -m abridgekv_amd.build` (there is no fallback path)")
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def check(rc: int, what: str) -> None:
    """Raise RuntimeError for a non-zero HIP error code returned by a kernel entry point."""
    if rc != 0:
        raise RuntimeError(f"{what} failed with HIP error {rc}")
