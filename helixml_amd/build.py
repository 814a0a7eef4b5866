"""Builds libhelix_hip.so (gfx950) in-tree with hipcc.

Each ``csrc/*.hip`` file (kernels and the C ABI) is compiled with hipcc and each ``host/*.cpp``
file (the native C++ host layer of ``include/helix/helix.hpp``) with g++, in parallel; all are
linked into ``helixml_amd/libhelix_hip.so``. The library has no torch dependency.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB = PKG / "libhelix_hip.so"
OBJDIR = PKG / "_build"

ARCH = os.environ.get("HELIX_HIP_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-munsafe-fp-atomics",
    # multiply-adds fuse only within one expression (explicit fmaf elsewhere), and
    # `#pragma clang fp contract(off)` is honoured where the reference's unfused f32 order must be
    # reproduced
    "-ffp-contract=on",
    # packed FP32 VALU ops are disabled: hipcc would otherwise form v_pk_* from scalar code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


HOST = PKG / "host"
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{INCLUDE}"]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(HOST.glob("*.cpp"))


def _compile(src: Path) -> Path:
    if src.suffix == ".cpp":
        obj = OBJDIR / (src.stem + ".host.o")
        cmd = [os.environ.get("CXX", "g++"), *CXX_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        obj = OBJDIR / (src.stem + ".o")
        cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed for {src.name}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compiles every HIP source and links libhelix_hip.so; returns its path."""
    OBJDIR.mkdir(exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
