"""The GPU decode kernels themselves (bigsmall_amd/csrc/bsck_decode.hip and
refcodec_decode.hip) run on the CPU under AddressSanitizer and UBSan, built
as host C++ with the SIMT emulation of bigsmall_amd/csrc/simt_cpu.h (one fiber
per lane, wavefront operations and barriers as switch points), driven by
tests/native/decode_fuzz.cpp; a second build at -O2 without instrumentation
decodes the clean blobs and a share of the corrupted ones.

Cases: clean blobs of every BSCK plane mode, state width, element size and
coder (rANS; tANS with its states at the stream head or in a u32 array), the
layout-version-2 golden blobs, and of the reference's three formats on both decode paths (wave-serial and
lane-per-chain), each of which must decode to its source; then thousands of
corrupted copies (single and multiple byte changes, biased to the headers,
tables and chunk tables, and truncations). A corrupted BSCK blob goes to the
kernel whenever the host header check passes; a corrupted reference-format
blob goes to the kernels with the descriptors the library's own host parser
makes from it, whenever that parser accepts it. Every access stays inside its
buffer, or the sanitizer fails the run. The same corruption sweeps run on the
GPU in smaller numbers (tests/test_gpu_bsck.py, tests/test_gpu_refcodecs.py).
The clean BSCK blobs are also decoded together in batched launches of up to
64 tasks, five times that, and 4,096, 4,097 and 4,200 (small ones), so that a
workgroup finds its task by one, two and three rounds of the wavefront vote
(4,096 / 4,097 being the boundary between two and three); and a task table out
of order sends a workgroup to an empty task, which must stop at its header.
"""
from __future__ import annotations

import re
import shutil
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle
from bigsmall_amd.codecs import _refstreams
from bigsmall_amd.codecs import bf16_chunked as bc

ROOT = Path(__file__).resolve().parents[1]
CLANG = "/opt/rocm/llvm/bin/clang++"


def _bf16(x: np.ndarray) -> np.ndarray:
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _fp8(x: np.ndarray) -> np.ndarray:
    """fp8 e4m3 bytes of x (torch's rounding)."""
    import torch
    return torch.from_numpy(x.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy().copy()


def _case(kind: int, clean: bool, n: int, eb: int, blob: bytes, extra: bytes = b"", want: bytes = b"") -> bytes:
    return struct.pack("<BBHQIQ", kind, int(clean), 0, n, eb, len(blob)) + blob + extra + (want if clean else b"")


def _ref_extra(plan) -> bytes:
    se, tab, bst, mb, mt = _refstreams._plan_arrays(plan, 0)
    ns, nb, nt = len(plan.se_streams), len(plan.buckets), max(1, len(plan.mant_freqs))
    return (struct.pack("<IIII", ns, nb, nt, tab.nbytes) + se.tobytes() + tab.tobytes() + bst.tobytes() + mb.tobytes()
            + mt.tobytes())


def _corrupt(rng, blob: bytes) -> bytes:
    b = bytearray(blob)
    r = rng.random()
    if r < 0.1 and len(b) > 1:                               # truncation
        return bytes(b[: int(rng.integers(0, len(b)))])
    for _ in range(1 if r < 0.7 else int(rng.integers(2, 6))):
        hi = min(len(b), 512) if rng.random() < 0.5 else len(b)  # half in the header / tables / chunk table
        p = int(rng.integers(0, hi))
        b[p] ^= int(rng.integers(1, 256))
    return bytes(b)


def _bsck_inputs(rng):
    g = _bf16(rng.standard_normal(3000) * 0.02)
    hz = _bf16(rng.standard_normal(5000) * 0.02)
    hz[rng.permutation(hz.size)[: hz.size // 2]] = 0
    norms = _bf16(1 + rng.standard_normal(4096) * 0.01)
    yield g, dict(lanes=128, steps=16)
    yield g[:200], dict(lanes=64, steps=16)
    yield _bf16(rng.standard_t(3, 9000) * 0.02), dict(lanes=256, steps=32)
    yield hz, dict(lanes=128, steps=16, mode=2)
    yield hz[:1500], dict(lanes=64, steps=32, mode=2)
    yield norms, dict(lanes=128, steps=16)                   # exact-value mode
    yield rng.integers(0, 65536, 2500).astype(np.uint16), dict(lanes=128, steps=16, mode=1)
    yield rng.integers(0, 256, 4000).astype(np.uint8), dict(lanes=128, steps=16)     # byte elements
    yield np.array([0x3F80], np.uint16), dict(lanes=64, steps=16)
    # three or more full chunks (interleaved output units and plane blocks) and a tail, every state width
    yield _bf16(rng.standard_normal(3 * 1024 + 700) * 0.02), dict(lanes=64, steps=16, mode=1)
    yield _bf16(rng.standard_normal(4 * 2048 + 5) * 0.02), dict(lanes=128, steps=16, mode=1)
    yield _bf16(rng.standard_normal(3 * 4096 + 300) * 0.02), dict(lanes=256, steps=16, mode=1)
    yield rng.integers(0, 40, 5 * 2048 + 77).astype(np.uint8), dict(lanes=128, steps=16)
    # long chunks: the ring pipelines run many blocks; uniform bytes need about one renorm word per
    # two elements, which empties the word ring faster than loads refill it
    yield rng.integers(0, 256, 3 * 8192 + 100).astype(np.uint8), dict(lanes=128, steps=64)
    hz2 = _bf16(rng.standard_normal(3 * 8192 + 33) * 0.02)
    hz2[rng.permutation(hz2.size)[: hz2.size // 2]] = 0
    yield hz2, dict(lanes=128, steps=64, mode=2)
    yield _bf16(rng.standard_normal(2 * 8192 + 9) * 0.02), dict(lanes=128, steps=64, mode=1)
    # fp8 exponent pairs (plane mode 3), every state width, with a tail
    f8 = _fp8(rng.standard_normal(2 * (3 * 2048 + 77)))
    yield f8, dict(lanes=128, steps=16, mode=3)
    yield f8[:2 * 700], dict(lanes=64, steps=16, mode=3)
    yield f8, dict(lanes=256, steps=16, mode=3)
    # tANS: every plane mode, state width and element kind, full chunks and tails, with the
    # initial states at the stream head (coder 2) and in the u32 array of earlier blobs (coder 1)
    tans = [(g, dict(lanes=128, steps=16)), (g[:200], dict(lanes=64, steps=16)),
            (_bf16(rng.standard_t(3, 9000) * 0.02), dict(lanes=256, steps=32)),
            (hz, dict(lanes=128, steps=16, mode=2)), (hz[:1500], dict(lanes=64, steps=32, mode=2)),
            (hz, dict(lanes=256, steps=16, mode=2)), (norms, dict(lanes=128, steps=16)),
            (rng.integers(0, 65536, 2500).astype(np.uint16), dict(lanes=128, steps=16, mode=1)),
            (rng.integers(0, 256, 4000).astype(np.uint8), dict(lanes=128, steps=16)),
            (rng.integers(0, 256, 3 * 8192 + 100).astype(np.uint8), dict(lanes=128, steps=64)),
            (hz2, dict(lanes=128, steps=64, mode=2)), (f8, dict(lanes=128, steps=16, mode=3)),
            (f8, dict(lanes=256, steps=16, mode=3)), (np.array([0x3F80], np.uint16), dict(lanes=64, steps=16)),
            # compact mode at ~20 bits per element (uniform words: 8-bit exponent classes plus
            # 8 plane bits), beyond the 12 per element the block-level ring refill provides
            (rng.integers(0, 65536, 3 * 8192 + 5).astype(np.uint16), dict(lanes=256, steps=32, mode=2)),
            (rng.integers(0, 65536, 2 * 8192 + 3).astype(np.uint16), dict(lanes=128, steps=64, mode=2)),
            # one symbol: no element bits, so a coder-2 stream is its head states alone
            (np.full(700, 0x3F80, np.uint16), dict(lanes=256, steps=16)),
            (np.full(300, 0x3F80, np.uint16), dict(lanes=64, steps=16))]
    for coder in (2, 1):
        for w, kw in tans:
            yield w, dict(kw, coder=coder)


def _ref_inputs(rng):
    yield "bf16_parallel_v1", _bf16(rng.standard_normal(1200) * 0.02), lambda w: oracle.par1_encode(w, 8)
    yield "bf16_parallel_v1", _bf16(rng.standard_t(3, 700) * 0.02), lambda w: oracle.par1_encode(w, 3)
    yield "bf16_se_tans", _bf16(rng.standard_normal(600) * 0.02), oracle.tans_encode
    yield "bf16_se_single_kernel", _bf16(rng.standard_normal(600) * 0.5), oracle.sk_encode
    hz = _bf16(rng.standard_normal(800) * 0.02)
    hz[rng.permutation(hz.size)[:400]] = 0
    yield "bf16_se_tans", hz, oracle.tans_encode


def _write_cases(path: Path, n_bsck: int, n_ref: int) -> dict:
    rng = np.random.default_rng(2024)
    cases, counts = [], {"bsck_clean": 0, "bsck_corrupt": 0, "ref_clean": 0, "ref_corrupt": 0, "ref_parser_refused": 0}
    bsck = [(w, bc.encode_array(w, **kw)) for w, kw in _bsck_inputs(rng)]
    # layout-version-2 blobs written by the earlier encoder (tests/golden/make_bsck_v2.py)
    v2 = np.load(Path(__file__).resolve().parent / "golden" / "bsck_v2_vectors.npz")
    bsck += [(v2[k], v2["blob_" + k[4:]].tobytes()) for k in v2.files if k.startswith("src_")]
    for w, blob in bsck:
        eb = w.dtype.itemsize
        cases.append(_case(0, True, w.size, eb, blob, want=w.tobytes()))
        counts["bsck_clean"] += 1
        for _ in range(n_bsck // len(bsck)):
            cases.append(_case(0, False, w.size, eb, _corrupt(rng, blob)))
            counts["bsck_corrupt"] += 1
    refs = list(_ref_inputs(rng))
    for codec, w, enc in refs:
        blob = enc(w)
        plan = _refstreams.PARSERS[codec](blob, w.size)
        for kind in (1, 2):                                   # wave-serial, lane per chain
            cases.append(_case(kind, True, w.size, 2, blob, _ref_extra(plan), w.tobytes()))
            counts["ref_clean"] += 1
        made = 0
        while made < n_ref // len(refs):
            bad = _corrupt(rng, blob)
            try:                                              # the host parse and table build, as in RefLaunch
                plan = _refstreams.PARSERS[codec](bad, w.size)
                extra = _ref_extra(plan) if plan.se_streams else None
            except ValueError:
                counts["ref_parser_refused"] += 1
                continue
            if extra is None:
                continue
            kind = 1 if made % 2 == 0 else 2
            cases.append(_case(kind, False, w.size, 2, bad, extra))
            counts["ref_corrupt"] += 1
            made += 1
    path.write_bytes(struct.pack("<II", 0x5A465342, len(cases)) + b"".join(cases))
    return counts


SANITIZE = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer",
            "-fsanitize-address-use-after-return=never"]


def _build(tmp_path: Path, flags: list[str], name: str) -> Path:
    exe = tmp_path / name
    csrc = ROOT / "bigsmall_amd" / "csrc"
    cmd = [CLANG, "-std=c++17", "-O2", "-g", "-pthread", "-DBS_SIMT_CPU", "-DBSCK_WAVES=4", *flags,
           "-I", str(ROOT / "include"), "-I", str(csrc),
           "-x", "c++", str(csrc / "bsck_decode.hip"), str(csrc / "refcodec_decode.hip"),
           str(ROOT / "tests" / "native" / "decode_fuzz.cpp"), "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


@pytest.mark.skipif(not Path(CLANG).exists() or shutil.which("make") is None, reason="needs ROCm's clang++")
def test_decode_kernels_under_sanitizers(tmp_path):
    oracle.build()
    exe = _build(tmp_path, SANITIZE, "decode_fuzz")
    cases = tmp_path / "cases.bin"
    counts = _write_cases(cases, n_bsck=3000, n_ref=2400)
    r = subprocess.run([str(exe), str(cases)], capture_output=True, text=True, timeout=1800,
                       env={"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1", "UBSAN_OPTIONS": "print_stacktrace=1"})
    print(counts, r.stdout, r.stderr[-3000:])
    assert r.returncode == 0, r.stdout + r.stderr[-3000:]
    batch, line = r.stdout.strip().splitlines()[-2:]
    assert "clean failed 0" in line, line
    assert counts["bsck_corrupt"] + counts["ref_corrupt"] >= 5000
    # every clean BSCK blob decoded in the batched launches (as they are, five times over,
    # and 4,096, 4,097 and 4,200 small ones), some from addresses with bit 31 set; the
    # out-of-order table's empty task was flagged at its header check; the clean
    # wave-serial reference cases decoded again in one batch with gaps between
    # the tasks' SE groups
    ok, failed, high, empty, gaps = (int(v) for v in re.findall(r"\d+", batch.replace("bit 31", "")))
    assert ok == 6 * counts["bsck_clean"] + 4096 + 4097 + 4200 and failed == 0 and high > 0, batch
    assert empty == 1 and gaps >= 2, batch


@pytest.mark.skipif(not Path(CLANG).exists() or shutil.which("make") is None, reason="needs ROCm's clang++")
def test_decode_kernels_optimised_without_instrumentation(tmp_path):
    """The same kernels at -O2 with no sanitizer: instrumentation changes what
    the optimiser may assume, and code that is only right when unoptimised (an
    LDS access moved across a wavefront barrier, say) shows here as a clean
    blob decoding wrong."""
    oracle.build()
    exe = _build(tmp_path, [], "decode_plain")
    cases = tmp_path / "cases.bin"
    _write_cases(cases, n_bsck=600, n_ref=480)
    r = subprocess.run([str(exe), str(cases)], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout + r.stderr[-3000:]
    assert "clean failed 0" in r.stdout.strip().splitlines()[-1]
