"""Build libbigsmall_hip.so (the decode engine's C-ABI library) in-tree.

HIP sources (csrc/*.hip) are compiled with hipcc for gfx950 only; host C++
sources (csrc/*.cpp) with g++. Output: bigsmall_amd/_lib/libbigsmall_hip.so.
Packed-FP32 instruction selection is disabled for all device code.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB = OUT_DIR / "libbigsmall_hip.so"
INC = PKG.parent / "include"

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]
CXX_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-pthread", "-Wall"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        sys.stderr.write(err + "\n")
        raise RuntimeError(f"build step failed: {' '.join(cmd)}")
    if err and os.environ.get("BIGSMALL_BUILD_VERBOSE"):
        sys.stderr.write(err + "\n")


def build(verbose: bool = False) -> Path:
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    cxx = shutil.which("g++") or "g++"
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    objs = []
    for src in sorted(CSRC.glob("*.hip")):
        o = obj_dir / (src.stem + ".hip.o")
        _run([hipcc, *HIP_FLAGS, "-I", str(INC), "-c", str(src), "-o", str(o)])
        objs.append(o)
    for src in sorted(CSRC.glob("*.cpp")):
        o = obj_dir / (src.stem + ".cpp.o")
        _run([cxx, *CXX_FLAGS, "-I", str(INC), "-c", str(src), "-o", str(o)])
        objs.append(o)
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-pthread", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
