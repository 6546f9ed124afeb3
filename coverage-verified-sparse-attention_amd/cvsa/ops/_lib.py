"""ctypes binding of libcvsa_hip.so (the C ABI declared in include/cvsa_hip.h).

The library is built in-tree by ``csrc/build.py`` (or ``__graft_entry__.build``)
and loaded once.  There is no fallback: every op in :mod:`cvsa.ops` raises if
the library is missing.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parents[1] / "libcvsa_hip.so"
ABI_VERSION = 14

CVSA_OK = 0
CVSA_ERR_INVALID = -1
CVSA_ERR_UNSUPPORTED = -2
CVSA_ERR_LAUNCH = -3
CVSA_ERR_WORKSPACE = -4

DTYPE_BF16 = 0
DTYPE_FP16 = 1
DTYPE_FP32 = 2

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

STEP_REUSE = 0
STEP_LAZY_CHECK = 1
STEP_SCORE = 2
STEP_FRESH = 3

SELECT_EXACT = 0
SELECT_QUEST = 1
SELECT_QUEST_LN = 2


class StepDesc(ctypes.Structure):
    """cvsa_step_desc (include/cvsa_hip.h), field for field."""
    _fields_ = [
        ("B", _i32), ("H_q", _i32), ("H_kv", _i32), ("D", _i32), ("block_size", _i32),
        ("W", _i32), ("budget", _i32), ("tau", _f32), ("out_dtype", _i32),
        ("q_stride_b", _i64), ("q_stride_h", _i64),
        ("k_cache", _p), ("v_cache", _p), ("num_blocks", _i64),
        ("block_tables", _p), ("bt_stride_b", _i64), ("context_lens", _p),
        ("page_indices", _p), ("n_per_head", _p), ("page_scores", _p), ("scores_cache", _p),
        ("check_accept", _p), ("accept", _p), ("coverage", _p), ("stats", _p), ("work", _p),
        ("workspace", _p), ("workspace_bytes", _sz),
        ("selector", _i32), ("quest_meta", _p), ("quest_ntok", _p), ("sel_scores", _p),
        ("spec_state", _p), ("sel_map", _p), ("sel_map_stride", _i64),
        ("approx_budget", _i32), ("approx_indices", _p),
    ]


# name -> (restype, argtypes); mirrors include/cvsa_hip.h
SIGNATURES = {
    "cvsa_last_error": (ctypes.c_char_p, []),
    "cvsa_abi_version": (ctypes.c_int, []),
    "cvsa_score_pages": (ctypes.c_int, [
        _p, _i64, _i64, _p, _i64, _p, _i64, _p,
        _i32, _i32, _i32, _i32, _i32, _i32, _p, _p]),
    "cvsa_select_topk": (ctypes.c_int, [
        _p, _i32, _i32, _i32, _p, _i32, _i32, _p, _p, _f32, _p, _p, _p]),
    "cvsa_select_or_keep": (ctypes.c_int, [
        _p, _p, _p, _i32, _i32, _i32, _p, _i32, _i32, _p, _p, _f32, _p, _p, _p, _p, _i32, _p]),
    "cvsa_select_or_keep_budgeted": (ctypes.c_int, [
        _p, _p, _p, _i32, _i32, _i32, _p, _i32, _p, _i32, _p, _p, _f32, _p, _p, _p, _p, _i32,
        _p]),
    "cvsa_select_budgeted": (ctypes.c_int, [
        _p, _p, _i32, _i32, _i32, _p, _i32, _f32, _p, _i32, _p, _p, _f32, _p, _p, _p]),
    "cvsa_adaptive_budgets": (ctypes.c_int, [
        _p, _i32, _i32, _i32, _p, _i32, _i32, ctypes.c_double, _p, _p]),
    "cvsa_check_coverage": (ctypes.c_int, [
        _p, _i32, _i32, _i32, _p, _i64, _p, _f32, _p, _p, _p]),
    "cvsa_decode_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "cvsa_workspace_init": (ctypes.c_int, [_p, _sz, _p]),
    "cvsa_sparse_decode": (ctypes.c_int, [
        _p, _i64, _i64, _p, _p, _i64, _p, _i64, _p,
        _p, _i64, _p, _i32,
        _i32, _i32, _i32, _i32, _i32, _i32,
        _p, _p, _p, _p, _i32, _p, _p, _sz, _p]),
    "cvsa_sparse_decode_noalloc": (ctypes.c_int, [
        _p, _i64, _i64, _p, _p, _i64, _p, _i64, _p,
        _p, _i64, _p, _i32,
        _i32, _i32, _i32, _i32, _i32, _i32,
        _p, _p, _p, _p, _i32, _p, _p]),
    "cvsa_sparse_decode_append": (ctypes.c_int, [
        _p, _i64, _i64, _p, _p, _i64, _p, _i64, _p,
        _p, _i64, _p, _i32,
        _i32, _i32, _i32, _i32, _i32, _i32,
        _p, _i32, _p, _p, _sz, _p, _p, _i64, _p, _p, _p, _p, _p]),
    "cvsa_dense_decode": (ctypes.c_int, [
        _p, _i64, _i64, _p, _p, _i64, _p, _i64, _p,
        _i32, _i32, _i32, _i32, _i32, _i32,
        _p, _p, _p, _p, _i32, _p, _p, _sz, _p]),
    "cvsa_verified_decode": (ctypes.c_int, [
        _p, _i64, _i64, _p, _p, _i64, _p, _i64, _p,
        _p, _i64, _p, _i32, _p,
        _i32, _i32, _i32, _i32, _i32, _i32,
        _p, _p, _p, _p, _i32, _p, _p, _sz, _p]),
    "cvsa_verified_decode_approx": (ctypes.c_int, [
        _p, _i64, _i64, _p, _p, _i64, _p, _i64, _p,
        _p, _i64, _p, _i32, _p, _p, _i64, _i32,
        _i32, _i32, _i32, _i32, _i32, _i32,
        _p, _p, _p, _p, _i32, _p, _p, _sz, _p]),
    "cvsa_compute_complement": (ctypes.c_int, [
        _p, _i64, _p, _p, _i32, _p, _i32, _i32, _i32, _p, _p, _p]),
    "cvsa_lse_merge": (ctypes.c_int, [
        _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _p, _i32, _p]),
    "cvsa_append_kv": (ctypes.c_int, [
        _p, _p, _i64, _p, _p, _i64, _p, _i64, _i32, _p, _p,
        _i32, _i32, _i32, _i32, _i32, _i32, _p]),
    "cvsa_quest_meta_update": (ctypes.c_int, [
        _p, _i64, _p, _i64, _p, _i32, _i32, _i32, _i32, _i32, _p, _p, _p]),
    "cvsa_quest_scores": (ctypes.c_int, [
        _p, _i64, _i64, _p, _i64, _p, _i64, _p, _i32, _i32, _i32, _i32, _i32, _i32, _p, _p]),
    "cvsa_quest_refresh_scores": (ctypes.c_int, [
        _p, _i64, _i64, _p, _i64, _p, _i64, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32,
        _p, _p, _p, _p]),
    "cvsa_step_workspace_bytes": (_sz, [ctypes.POINTER(StepDesc)]),
    "cvsa_step_plan_create": (ctypes.c_int, [ctypes.POINTER(StepDesc), ctypes.POINTER(_p)]),
    "cvsa_step_plan_run": (ctypes.c_int, [_p, _i32, _p, _p, _p]),
    "cvsa_step_plan_run_append": (ctypes.c_int, [_p, _p, _p, _p, _p, _i64, _p, _p, _p, _p,
                                                  _p]),
    "cvsa_step_plan_destroy": (None, [_p]),
    "cvsa_step_plan_selection_changed": (ctypes.c_int, [_p]),
}

_LIB = None


class CVSAError(RuntimeError):
    """A libcvsa_hip entry point refused a call or a launch failed."""


def load() -> ctypes.CDLL:
    """Load libcvsa_hip.so once; raise if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise CVSAError(
            f"{LIB_PATH} is missing: build it with csrc/build.py (or "
            "__graft_entry__.build()); the CVSA ops have no non-HIP path")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.cvsa_abi_version()
    if ver != ABI_VERSION:
        raise CVSAError(f"libcvsa_hip ABI version {ver}, expected {ABI_VERSION}; rebuild it")
    _LIB = lib
    return lib


def check(rc: int, what: str) -> None:
    """Turn a CVSA status code into the matching Python exception."""
    if rc == CVSA_OK:
        return
    msg = (load().cvsa_last_error() or b"").decode(errors="replace")
    if rc == CVSA_ERR_INVALID:
        raise ValueError(f"{what}: {msg}")
    if rc == CVSA_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise CVSAError(f"{what} failed (status {rc}): {msg}")
