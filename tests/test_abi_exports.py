"""The C-ABI library loads without a GPU and exports exactly what
include/cvsa_hip.h declares, with the ctypes table in step with it."""
import ctypes
import os
import re

import pytest

from cvsa.ops import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "cvsa_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"^\s*(?:const\s+)?\w+\s*\*?\s*(cvsa_\w+)\s*\(([^)]*)\)\s*;", text,
                         flags=re.M):
        args = [a.strip() for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        decls[m.group(1)] = args
    return decls


def _lib_or_skip():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libcvsa_hip.so not built")
    try:
        return _lib.load()
    except OSError as e:  # no HIP runtime on this host
        pytest.skip(f"HIP runtime not loadable: {e}")


def test_header_and_ctypes_table_agree():
    decls = _declared()
    assert len(decls) >= 14
    assert set(decls) == set(_lib.SIGNATURES)
    for name, args in decls.items():
        assert len(args) == len(_lib.SIGNATURES[name][1]), name


def test_library_exports_every_declared_symbol():
    lib = _lib_or_skip()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.cvsa_abi_version() == _lib.ABI_VERSION


def test_errors_are_reported_without_gpu_work():
    """Argument validation runs on the host before any launch."""
    lib = _lib_or_skip()
    rc = lib.cvsa_select_topk(None, 1, 1, 8, None, 16, 3, None, None, 0.9, None, None, None)
    assert rc == _lib.CVSA_ERR_INVALID
    assert b"select_topk" in lib.cvsa_last_error()
    rc = lib.cvsa_decode_workspace_bytes(1, 32, 8, 128, 64, 8192, 1)
    assert rc > 0


def test_decode_workspace_layout_is_fixed():
    """Every decode workspace starts with the same 18 KiB counter area
    (4096 head counters and 512 group counters of the two-level merge, 4
    bytes each) followed by whole partial rows of G x (D + 4)
    fp32, so launches of any B * H_kv can share one workspace: the counters
    of one launch never overlap the partial rows of another.  Head dimensions
    outside {32, 64, 128, 256} have no workspace (0)."""
    lib = _lib_or_skip()
    seen = 0
    for D in (32, 64, 128, 256):
        for B in (1, 2, 3, 16, 32, 64):
            for H_kv, G in ((8, 4), (4, 7), (8, 8), (1, 1)):
                for max_sel, W, all_pages in ((1024, 8192, 0), (128, 512, 1), (64, 2048, 0),
                                              (0, 512, 1)):
                    n = lib.cvsa_decode_workspace_bytes(B, H_kv * G, H_kv, D, max_sel, W,
                                                        all_pages)
                    if n == 0:
                        continue
                    seen += 1
                    assert n > 18432 and (n - 18432) % (G * (D + 4) * 4) == 0, (B, H_kv, G, n)
    assert seen > 60
    assert lib.cvsa_decode_workspace_bytes(1, 32, 8, 96, 64, 8192, 1) == 0


def _step_desc(**over):
    """A well-formed step descriptor over fake (never dereferenced) pointers."""
    fake = iter(range(1 << 20, 1 << 30, 1 << 16))
    d = dict(B=1, H_q=32, H_kv=8, D=128, block_size=16, W=512, budget=128, tau=0.9,
             out_dtype=_lib.DTYPE_BF16, q_stride_b=32 * 128, q_stride_h=128, num_blocks=600,
             bt_stride_b=512)
    for name in ("k_cache", "v_cache", "block_tables", "context_lens", "page_indices",
                 "n_per_head", "page_scores", "check_accept", "accept", "coverage"):
        d[name] = next(fake)
    d.update(over)
    desc = _lib.StepDesc(**{k: v for k, v in d.items() if k != "workspace_bytes"})
    need = _lib.load().cvsa_step_workspace_bytes(ctypes.byref(desc))
    desc.workspace = next(fake) * 256 if need else None
    desc.workspace_bytes = d.get("workspace_bytes", need)
    return desc


def test_step_plan_validates_on_the_host():
    lib = _lib_or_skip()
    h = ctypes.c_void_p()
    desc = _step_desc()
    assert lib.cvsa_step_workspace_bytes(ctypes.byref(desc)) == max(
        lib.cvsa_decode_workspace_bytes(1, 32, 8, 128, 128, 512, 0),
        lib.cvsa_decode_workspace_bytes(1, 32, 8, 128, 128, 512, 1))
    assert lib.cvsa_step_plan_create(ctypes.byref(desc), ctypes.byref(h)) == _lib.CVSA_OK
    assert h.value
    # run-time argument errors are reported before anything is enqueued
    assert lib.cvsa_step_plan_run(h, 1, None, 1 << 20, None) == _lib.CVSA_ERR_INVALID
    assert lib.cvsa_step_plan_run(h, 7, 1 << 20, 1 << 20, None) == _lib.CVSA_ERR_INVALID
    assert b"kind" in lib.cvsa_last_error()
    assert lib.cvsa_step_plan_run(h, 0, (1 << 20) + 2, 1 << 20, None) == _lib.CVSA_ERR_INVALID
    assert lib.cvsa_step_plan_selection_changed(h) == _lib.CVSA_OK  # host state only
    assert lib.cvsa_step_plan_selection_changed(None) == _lib.CVSA_ERR_INVALID
    lib.cvsa_step_plan_destroy(h)
    # a valid selection map is accepted
    ok = _step_desc(sel_map=1 << 26, sel_map_stride=512)
    assert lib.cvsa_step_plan_create(ctypes.byref(ok), ctypes.byref(h)) == _lib.CVSA_OK
    lib.cvsa_step_plan_destroy(h)
    # any KV-head count is accepted (here one that is neither 1, 2, 4, 8 nor 16)
    ok = _step_desc(H_kv=3, H_q=12)
    assert lib.cvsa_step_plan_create(ctypes.byref(ok), ctypes.byref(h)) == _lib.CVSA_OK
    lib.cvsa_step_plan_destroy(h)
    cases = [(dict(budget=513), _lib.CVSA_ERR_INVALID, b"budget"),
             (dict(H_kv=3, H_q=10), _lib.CVSA_ERR_INVALID, b"head counts"),
             (dict(D=96), _lib.CVSA_ERR_UNSUPPORTED, b"D=96"),
             (dict(block_size=12), _lib.CVSA_ERR_UNSUPPORTED, b"block_size=12"),
             (dict(block_size=256), _lib.CVSA_ERR_UNSUPPORTED, b"block_size=256"),
             (dict(bt_stride_b=100), _lib.CVSA_ERR_INVALID, b"stride"),
             (dict(coverage=None), _lib.CVSA_ERR_INVALID, b"null"),
             (dict(out_dtype=5), _lib.CVSA_ERR_INVALID, b"dtype"),
             (dict(workspace_bytes=1024), _lib.CVSA_ERR_WORKSPACE, b"workspace"),
             (dict(selector=3), _lib.CVSA_ERR_INVALID, b"selector"),
             (dict(selector=_lib.SELECT_QUEST_LN), _lib.CVSA_ERR_INVALID, b"quest_meta"),
             (dict(selector=_lib.SELECT_QUEST, quest_meta=1 << 24, quest_ntok=1 << 25),
              _lib.CVSA_ERR_INVALID, b"sel_scores"),
             # selection map rows: at least W bytes, a multiple of 16, 16-byte aligned
             (dict(sel_map=1 << 26, sel_map_stride=496), _lib.CVSA_ERR_INVALID, b"sel_map"),
             (dict(sel_map=1 << 26, sel_map_stride=520), _lib.CVSA_ERR_INVALID, b"sel_map"),
             (dict(sel_map=(1 << 26) + 8, sel_map_stride=512), _lib.CVSA_ERR_INVALID,
              b"sel_map")]
    for over, code, word in cases:
        h = ctypes.c_void_p()
        rc = lib.cvsa_step_plan_create(ctypes.byref(_step_desc(**over)), ctypes.byref(h))
        assert rc == code, over
        assert word in lib.cvsa_last_error(), (over, lib.cvsa_last_error())
        assert not h.value
