"""Builds the C++ host-layer test program (tests/cpp/helix_host_tests) with g++: test_host.cpp
linked against helixml_amd/libhelix_hip.so and the oracle's liboracle.so (test infrastructure).
Run by __graft_entry__.build() after the library and the oracle are built."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
EXE = HERE / "helix_host_tests"


def build() -> Path:
    lib_dir = ROOT / "helixml_amd"
    ora_dir = ROOT / "oracle"
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-Wall", f"-I{ROOT / 'include'}", f"-I{ROOT / 'helixml_amd' / 'host'}",
           str(HERE / "test_host.cpp"), "-o", str(EXE),
           f"-L{lib_dir}", "-lhelix_hip", f"-L{ora_dir}", "-l:liboracle.so",
           f"-Wl,-rpath,{lib_dir}", f"-Wl,-rpath,{ora_dir}",
           # the box's copy of the tree sits at another path: also search relative to the binary
           "-Wl,-rpath,$ORIGIN/../../helixml_amd", "-Wl,-rpath,$ORIGIN/../../oracle"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building {EXE.name} failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return EXE


if __name__ == "__main__":
    print(build())
