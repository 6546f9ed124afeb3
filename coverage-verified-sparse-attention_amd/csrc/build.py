"""Build libcvsa_hip.so for gfx950 from the sources in this directory.

Every ``*.hip`` / ``*.cpp`` file is compiled to an object under ``../_build``
and linked into ``../cvsa/libcvsa_hip.so`` (the path the ctypes loader in
``cvsa/ops/_lib.py`` opens).  Always rebuilds; hipcc cross-compiles without a
GPU.

    python build.py [--jobs N] [--verbose]
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG_ROOT = HERE.parent
BUILD_DIR = PKG_ROOT / "_build"
LIB_PATH = PKG_ROOT / "cvsa" / "libcvsa_hip.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-command-line-argument",
    # Keep the compiler from forming packed fp32 VALU ops.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm install required to build libcvsa_hip.so)")


def _sources() -> list[Path]:
    return sorted(list(HERE.glob("*.hip")) + list(HERE.glob("*.cpp")))


def _compile(hipcc: str, src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".hip":
        cmd[1:1] = ["-x", "hip"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compiling {src.name} failed:\n{res.stdout}\n{res.stderr}")
    noisy = [ln for ln in res.stderr.splitlines()
             if ln.strip() and "packed-fp32-ops" not in ln]
    if noisy and verbose:
        print("\n".join(noisy), file=sys.stderr)
    return obj


def build(jobs: int = 4, verbose: bool = False) -> Path:
    hipcc = _hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = _sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s, verbose), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"linking libcvsa_hip.so failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    path = build(args.jobs, args.verbose)
    print(f"built {path}")


if __name__ == "__main__":
    main()
