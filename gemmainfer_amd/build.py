"""Builds libgemmainfer_amd.so (the C-ABI library) for gfx950 with hipcc.

Usage: ``python -m gemmainfer_amd.build`` (or ``build()`` from Python).  Each
``csrc/*.hip`` file compiles to an object in parallel; the objects link into
``gemmainfer_amd/lib/libgemmainfer_amd.so``.  No GPU is needed: hipcc cross
compiles for the MI355X (gfx950) here.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
LIBNAME = "libgemmainfer_amd.so"
OBJDIR = PKG / "_build"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-FP32 VALU forms are kept out of every kernel (the compiler would
# otherwise fuse scalar fp32 pairs into them); the host pass ignores the flag.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep small private arrays in registers: moved to LDS they cost a full
    # vmem drain and an LDS round trip per element
    "-mllvm", "-disable-promote-alloca-to-lds",
]


def lib_path() -> Path:
    return LIBDIR / LIBNAME


def _compile(src: Path) -> Path:
    obj = OBJDIR / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{out}")
    if out.strip():
        print(out, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every csrc/*.hip and link the shared library; returns its path."""
    OBJDIR.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIBDIR / (LIBNAME + ".tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, lib_path())
    if verbose:
        print(f"built {lib_path()} from {len(sources)} sources")
    return lib_path()


if __name__ == "__main__":
    build()
