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
