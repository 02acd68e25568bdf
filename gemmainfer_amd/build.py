"""Builds libgemmainfer_amd.so (the C-ABI library) for gfx950 with hipcc.

Usage: ``python -m gemmainfer_amd.build`` (or ``build()`` from Python).  Each
``csrc/*.hip`` file compiles to an object in parallel; the objects link into
``gemmainfer_amd/lib/libgemmainfer_amd.so``.  No GPU is needed: hipcc cross
compiles for the MI355X (gfx950) here.

``python -m gemmainfer_amd.build --timeline`` builds the measurement variant
``lib/libgemmainfer_amd_timeline.so`` (the same sources with -DGI_TIMELINE:
the decode kernel records per-workgroup phase stamps, see
include/gemmainfer_amd_probe.h); the product library never contains it.
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
TIMELINE_LIBNAME = "libgemmainfer_amd_timeline.so"
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


def lib_path(timeline: bool = False) -> Path:
    return LIBDIR / (TIMELINE_LIBNAME if timeline else LIBNAME)


def _compile(src: Path, timeline: bool = False) -> Path:
    objdir = OBJDIR.with_name(OBJDIR.name + "_timeline") if timeline else OBJDIR
    obj = objdir / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *(["-DGI_TIMELINE"] if timeline else []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{out}")
    if out.strip():
        print(out, file=sys.stderr)
    return obj


def build(verbose: bool = True, timeline: bool = False) -> Path:
    """Compile every csrc/*.hip and link the shared library; returns its path."""
    (OBJDIR.with_name(OBJDIR.name + "_timeline") if timeline else OBJDIR).mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(lambda src: _compile(src, timeline), sources))
    out = lib_path(timeline)
    tmp = out.with_name(out.name + ".tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} from {len(sources)} sources")
    return out


if __name__ == "__main__":
    build(timeline="--timeline" in sys.argv[1:])
