"""Write BSCK layout-version-2 blobs (the chunk-contiguous layout of the
engine's earlier releases) as golden vectors for the decoders' v2 path.

The version-2 encoder no longer exists in the tree, so this script takes its
source from the repository's own history (commit 31181fa^, the last one with
layout version 2: bigsmall_amd/csrc/bsck_encode.cpp and include/bigsmall_hip.h),
builds it with g++ into a temporary directory and encodes seeded inputs with
it. Output: tests/golden/bsck_v2_vectors.npz, data only (uint16/uint8 source
arrays and the blobs as uint8 arrays, plus each case's encoder arguments).

Usage:  python tests/golden/make_bsck_v2.py   (needs git history and g++)
"""
from __future__ import annotations

import ctypes
import subprocess
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
OUT = Path(__file__).resolve().parent / "bsck_v2_vectors.npz"
REV = "31181fa^"


def _bf16(x: np.ndarray) -> np.ndarray:
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _build(tmp: Path) -> ctypes.CDLL:
    for rel in ("bigsmall_amd/csrc/bsck_encode.cpp", "include/bigsmall_hip.h"):
        dst = tmp / rel
        dst.parent.mkdir(parents=True, exist_ok=True)
        dst.write_bytes(subprocess.run(["git", "show", f"{REV}:{rel}"], cwd=ROOT, check=True,
                                       capture_output=True).stdout)
    so = tmp / "libv2enc.so"
    subprocess.run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-pthread",
                    str(tmp / "bigsmall_amd/csrc/bsck_encode.cpp"), "-o", str(so)], check=True)
    L = ctypes.CDLL(str(so))
    L.bs_chunk_encode_bound.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                        ctypes.POINTER(ctypes.c_uint64)]
    L.bs_chunk_encode.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                  ctypes.c_uint32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_uint64,
                                  ctypes.POINTER(ctypes.c_uint64), ctypes.c_int]
    return L


def _encode(L, a: np.ndarray, lanes: int, steps: int, mode: int) -> bytes:
    a = np.ascontiguousarray(a)
    bound = ctypes.c_uint64()
    assert L.bs_chunk_encode_bound(a.size, a.itemsize, lanes, steps, ctypes.byref(bound)) == 0
    out = np.zeros(bound.value, np.uint8)
    n = ctypes.c_uint64()
    rc = L.bs_chunk_encode(a.ctypes.data, a.size, a.itemsize, lanes, steps, mode, out.ctypes.data, bound.value,
                           ctypes.byref(n), 2)
    assert rc == 0, rc
    blob = out[: n.value].tobytes()
    assert blob[:5] == b"BSCK\x02", blob[:8]
    return blob


def main() -> None:
    rng = np.random.default_rng(2)
    hz = _bf16(rng.standard_normal(9000) * 0.02)
    hz[rng.permutation(hz.size)[:4500]] = 0
    cases = [
        ("dense_128", _bf16(rng.standard_normal(3 * 2048 + 300) * 0.02), 128, 16, 1),
        ("dense_64", _bf16(rng.standard_normal(5 * 1024 + 7) * 0.02), 64, 16, 1),
        ("dense_256", _bf16(rng.standard_t(3, 2 * 4096 + 99) * 0.02), 256, 16, 1),
        ("compact", hz, 128, 16, 2),
        ("exact", _bf16(1.0 + rng.standard_normal(4096) * 0.01), 128, 16, 0),
        ("bytes", rng.integers(0, 40, 3 * 2048 + 5).astype(np.uint8), 128, 16, -1),
        ("one", np.array([0x3F80], np.uint16), 64, 16, -1),
    ]
    out = {}
    with tempfile.TemporaryDirectory() as d:
        L = _build(Path(d))
        for name, a, lanes, steps, mode in cases:
            out[f"src_{name}"] = a
            out[f"blob_{name}"] = np.frombuffer(_encode(L, a, lanes, steps, mode), np.uint8)
            out[f"args_{name}"] = np.array([lanes, steps, mode], np.int64)
            print(f"{name}: n={a.size} blob {out[f'blob_{name}'].size} bytes")
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
