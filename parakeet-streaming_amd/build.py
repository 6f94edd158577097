"""Build the gfx950 paged KV-cache library in-tree.

Produces ``parakeet_amd/libparakeet_paged.so`` next to the Python package that
loads it.  The HIP kernels are compiled with hipcc for gfx950 only; the host page
pool and error helpers are plain C++ (g++).  Run ``python build.py`` or call
``build()``; every call recompiles.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = REPO / "include"
BUILD_DIR = HERE / "_build"
CHECKS = REPO / "tests" / "native"
LIB_PATH = HERE / "parakeet_amd" / "libparakeet_paged.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ARCH = "gfx950"

# Packed FP32 instructions are disabled for all device code of this library.
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra"]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout)
        sys.stderr.write(res.stderr)
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}")
    if verbose and (res.stdout or res.stderr):
        # hipcc's host pass warns that it does not know the packed-fp32 feature
        lines = [
            ln
            for ln in (res.stdout + res.stderr).splitlines()
            if "packed-fp32-ops" not in ln and ln.strip()
        ]
        if lines:
            print("\n".join(lines), flush=True)


def build(verbose: bool = False) -> Path:
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    inc = [f"-I{INCLUDE}", f"-I{CSRC}"]
    objs: list[Path] = []

    for name in ("paged_kernels.hip", "conv_kernels.hip", "frontend_kernels.hip", "decode_kernels.hip"):
        obj = BUILD_DIR / (Path(name).stem + ".o")
        _run([HIPCC, *HIP_FLAGS, *inc, "-x", "hip", "-c", str(CSRC / name), "-o", str(obj)], verbose)
        objs.append(obj)

    for name in ("page_pool.cpp", "pk_common.cpp"):
        obj = BUILD_DIR / (Path(name).stem + ".o")
        _run([CXX, *CXX_FLAGS, *inc, "-c", str(CSRC / name), "-o", str(obj)], verbose)
        objs.append(obj)

    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, LIB_PATH)
    build_checks(verbose)
    return LIB_PATH


def build_checks(verbose: bool = False) -> list[Path]:
    """The stand-alone GPU check programs of tests/native (run by the GPU tests)."""
    out_dir = CHECKS / "_build"
    out_dir.mkdir(parents=True, exist_ok=True)
    built = []
    for src in sorted(CHECKS.glob("*.hip")):
        exe = out_dir / src.stem
        _run([HIPCC, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-x", "hip", str(src), "-o", str(exe)], verbose)
        built.append(exe)
    return built


def clean() -> None:
    shutil.rmtree(BUILD_DIR, ignore_errors=True)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
