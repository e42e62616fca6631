"""The GPU zstd decoder's core (bigsmall_amd/csrc/zstd_core.h) built for the
CPU under AddressSanitizer and UBSan and checked against libzstd: round trips
over data kinds and levels -5..22, and 4,800 corrupted frames, each of which
must decode to libzstd's bytes or be refused, with no access outside its
buffers (tests/native/zstd_core_check.cpp). Built with ROCm's clang++, every
frame also runs through the GPU's 64-lane team (each lane a fiber of
bigsmall_amd/csrc/simt_cpu.h, sync() the workgroup barrier), which must give
the one-lane team's bytes and error code on every frame; with only g++ the
one-lane team runs alone. The GPU runs the same code (tests/test_gpu_zstd.py)."""
from __future__ import annotations

import ctypes.util
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CLANG = "/opt/rocm/llvm/bin/clang++"


@pytest.mark.skipif(shutil.which("g++") is None or ctypes.util.find_library("zstd") is None,
                    reason="needs g++ and libzstd")
def test_zstd_core_round_trips_and_corruptions(tmp_path):
    import ctypes
    lib = ctypes.CDLL(ctypes.util.find_library("zstd"))._name
    exe = tmp_path / "zstd_core_check"
    team64 = Path(CLANG).exists()
    build = ([CLANG, "-O2", "-DBS_ZSTD_TEAM64", "-fsanitize-address-use-after-return=never"] if team64
             else ["g++", "-O1"])
    build += ["-g", "-std=c++17", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
              "-Wno-unknown-pragmas", str(ROOT / "tests/native/zstd_core_check.cpp"), "-o", str(exe)]
    path = Path(lib) if Path(lib).is_absolute() else None
    if path is None:                              # link the shared object by its soname
        for d in ("/usr/lib/x86_64-linux-gnu", "/usr/lib64", "/usr/lib", "/lib/x86_64-linux-gnu"):
            if (Path(d) / lib).exists():
                path = Path(d) / lib
                break
    if path is None:
        pytest.skip(f"cannot locate {lib}")
    subprocess.run(build + [str(path)], check=True, capture_output=True, timeout=300)
    r = subprocess.run([str(exe), "600"], capture_output=True, text=True, timeout=900,
                       env={"ASAN_OPTIONS": "detect_leaks=0", "UBSAN_OPTIONS": "print_stacktrace=1"})
    print(r.stdout, r.stderr[-2000:])
    assert r.returncode == 0, r.stdout + r.stderr[-2000:]
    assert "failed 0" in r.stdout and "decoded differently 0" in r.stdout
    if team64:
        assert "64-lane team differs from one lane on 0 frames" in r.stdout
