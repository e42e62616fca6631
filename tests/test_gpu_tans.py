"""GPU parity of the BSCK decoder's tANS coder, fp8 exponent-pair mode and
layout-version-2 path (bf16_chunked_tans_v1 / fp8_chunked_tans_v1, and
fp8_chunked_v1's pair mode).

Bar: bit-exact. Every case checks the GPU output == the source bytes (md5)
and == the oracle's CPU decode of the same blob. Also: the hand-built tANS
blob whose decode follows from its table (tests/test_bsck_formats_cpu.py),
one batched launch mixing both coders and every plane mode, corrupted tANS
blobs (each decodes to something or raises, never faults), and the v2
golden blobs. tANS runs with its initial states at the stream head (coder
2, what the encoder writes by default) and in the u32 state array of
earlier blobs (coder 1).
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _bf16(x: np.ndarray) -> np.ndarray:
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _fp8(x: np.ndarray) -> np.ndarray:
    import torch
    return torch.from_numpy(x.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy().copy()


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch_gpu():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    oracle.build()
    return torch


def _check(words, label, **kw):
    from bigsmall_amd.codecs import bf16_chunked as bc
    _say(f"[tans] {label} n={words.size} {kw}")
    blob = bc.encode_array(words, **kw)
    eb = words.dtype.itemsize
    gpu = bc.decode(blob, {}, words.size, elem_bytes=eb)
    assert hashlib.md5(gpu).hexdigest() == hashlib.md5(words.tobytes()).hexdigest(), label
    assert gpu == oracle.chunk_decode(blob, words.size, eb), label
    return blob


@pytest.mark.parametrize("coder", [2, 1])
@pytest.mark.parametrize("lanes", [64, 128, 256])
@pytest.mark.parametrize("n", [1, 63, 64, 65, 129, 4097, 65536 * 3 + 1000, 1 << 20])
def test_tans_gaussian_sizes(torch_gpu, n, lanes, coder):
    rng = np.random.default_rng(n + lanes)
    blob = _check(_bf16(rng.standard_normal(n) * 0.02), f"gauss{n}", steps=64, lanes=lanes, coder=coder)
    assert blob[28] == coder


@pytest.mark.parametrize("lanes", [64, 128, 256])
@pytest.mark.parametrize("mode", [-1, 1, 2])
@pytest.mark.parametrize("steps", [16, 128, 432])
def test_tans_modes_and_steps(torch_gpu, mode, steps, lanes):
    rng = np.random.default_rng(steps + 7 * mode + lanes)
    w = _bf16(rng.standard_normal(300_007) * 0.02)
    if mode == 2:
        w[rng.permutation(w.size)[: w.size // 2]] = 0
    blob = _check(w, f"mode{mode}", steps=steps, mode=mode, lanes=lanes, coder=2)
    assert blob[28] == 2


@pytest.mark.parametrize("coder", [0, 1, 2])
@pytest.mark.parametrize("lanes", [64, 128, 256])
def test_symbol_models(torch_gpu, coder, lanes):
    """Heavy tails, every word value, norms (exact values), one symbol,
    fp8 bytes and fp8 exponent pairs (with and without a partial chunk)."""
    rng = np.random.default_rng(100 + lanes + coder)
    _check(_bf16(rng.standard_t(3, 250_000) * 0.02), "studentt", steps=64, lanes=lanes, coder=coder)
    _check(rng.integers(0, 65536, 100_000).astype(np.uint16), "uniform words", steps=64, mode=1, lanes=lanes,
           coder=coder)
    _check(_bf16(1.0 + rng.standard_normal(4096 * 3) * 0.01), "norms", steps=16, lanes=lanes, coder=coder)
    _check(np.full(70_000, 0x3F80, np.uint16), "one value", steps=64, lanes=lanes, coder=coder)
    f8 = _fp8(rng.standard_normal(2 * 150_001))
    _check(f8, "fp8 bytes", steps=64, mode=0, lanes=lanes, coder=coder)
    blob = _check(f8, "fp8 pairs", steps=64, mode=3, lanes=lanes, coder=coder)
    assert blob[6] == 3
    _check(f8[: 2 * (lanes * 64) * 3], "fp8 pairs, whole chunks", steps=64, mode=3, lanes=lanes, coder=coder)
    _check(rng.integers(0, 256, 2 * 40_000).astype(np.uint8), "uniform bytes as pairs", steps=16, mode=3,
           lanes=lanes, coder=coder)


@pytest.mark.parametrize("coder", [2, 1])
@pytest.mark.parametrize("lanes", [64, 128, 256])
def test_compact_tans_beyond_the_refill_bound(torch_gpu, lanes, coder):
    """Compact chunks that take ~20 bits per element (uniform words: 8-bit
    exponent classes plus 8 plane bits), beyond the 12 per element the
    block-level ring refill provides: the steps land the rest themselves.
    Short and long chunks, with a partial chunk, and a tensor mixing such
    stretches with half-zero ones."""
    rng = np.random.default_rng(700 + lanes + coder)
    w = rng.integers(0, 65536, 400_003).astype(np.uint16)
    for steps in (16, 432):
        blob = _check(w, f"uniform compact steps={steps}", steps=steps, mode=2, lanes=lanes, coder=coder)
        assert blob[6] == 2 and blob[28] == coder
    mixed = _bf16(rng.standard_normal(600_000) * 0.02)
    mixed[rng.permutation(mixed.size)[:300_000]] = 0
    mixed[200_000:260_000] = rng.integers(0, 65536, 60_000).astype(np.uint16)
    _check(mixed, "mixed compact", steps=64, mode=2, lanes=lanes, coder=coder)


def test_hand_built_tans_blob(torch_gpu):
    from bigsmall_amd.codecs import bf16_chunked as bc
    from test_bsck_formats_cpu import hand_built_tans
    for seed in range(4):
        for coder in (1, 2):
            blob, want = hand_built_tans(seed, coder=coder)
            _say(f"[tans] hand-built blob {seed}, coder {coder}")
            assert bc.decode(blob, {}, want.size) == want.tobytes()


def test_layout_version_2_golden_blobs(torch_gpu):
    from bigsmall_amd.codecs import bf16_chunked as bc
    z = np.load(GOLDEN / "bsck_v2_vectors.npz")
    for k in z.files:
        if not k.startswith("src_"):
            continue
        src, blob = z[k], z["blob_" + k[4:]].tobytes()
        _say(f"[tans] v2 blob {k[4:]}")
        assert bc.decode(blob, {}, src.size, elem_bytes=src.dtype.itemsize) == src.tobytes(), k


def test_batch_mixing_coders_and_modes(torch_gpu):
    """One launch: rANS and tANS blobs of every plane mode and element kind,
    and v2 blobs, each decoded bit-exact into its own buffer."""
    torch = torch_gpu
    from bigsmall_amd.codecs import bf16_chunked as bc
    from bigsmall_amd.device import ChunkBatch, ChunkJob, StatusWord, upload_bytes
    rng = np.random.default_rng(5)
    items = []
    for coder in (0, 1, 2):
        g = _bf16(rng.standard_normal(80_001) * 0.02)
        hz = g.copy()
        hz[rng.permutation(hz.size)[: hz.size // 2]] = 0
        f8 = _fp8(rng.standard_normal(2 * 33_333))
        for w, kw in [(g, dict(mode=1)), (hz, dict(mode=2)), (_bf16(1 + rng.standard_normal(5000) * 0.01), {}),
                      (f8, dict(mode=3)), (f8, dict(mode=0)), (g[:77], {})]:
            items.append((w, bc.encode_array(w, steps=32, coder=coder, **kw)))
    z = np.load(GOLDEN / "bsck_v2_vectors.npz")
    items += [(z[k], z["blob_" + k[4:]].tobytes()) for k in z.files if k.startswith("src_")]
    dev = torch.device("cuda")
    d = [upload_bytes(b, dev) for _, b in items]
    outs = [torch.empty(w.nbytes, dtype=torch.uint8, device=dev) for w, _ in items]
    jobs = [ChunkJob(db.data_ptr(), len(b), o.data_ptr(), w.size, bc.info(b).n_chunks, bc.info(b).plane_mode)
            for db, (w, b), o in zip(d, items, outs)]
    st = StatusWord(dev)
    _say(f"[tans] batch of {len(jobs)} blobs, both coders, every plane mode")
    ChunkBatch(jobs, dev).launch(st)
    torch.cuda.synchronize()
    st.check("mixed batch")
    for i, ((w, _), o) in enumerate(zip(items, outs)):
        assert o.cpu().numpy().tobytes() == w.tobytes(), i


@pytest.mark.parametrize("coder", [2, 1])
@pytest.mark.parametrize("mode", [1, 2, 3])
def test_corrupted_tans_blobs_never_fault(torch_gpu, mode, coder):
    """Single-byte corruptions biased to the header, tables and chunk table:
    each decodes (to anything) or raises ValueError / DecodeError."""
    from bigsmall_amd.codecs import bf16_chunked as bc
    from bigsmall_amd.exceptions import DecodeError
    rng = np.random.default_rng(40 + mode + 10 * coder)
    if mode == 3:
        w = _fp8(rng.standard_normal(2 * 20_000))
    else:
        w = _bf16(rng.standard_normal(40_000) * 0.02)
        if mode == 2:
            w[rng.permutation(w.size)[:20_000]] = 0
    blob = bc.encode_array(w, steps=16, mode=mode, coder=coder)
    _say(f"[tans] corruption sweep mode {mode}, coder {coder}, blob {len(blob)} bytes")
    raised = decoded = 0
    for _ in range(120):
        b = bytearray(blob)
        p = int(rng.integers(0, min(len(b), 17_000))) if rng.random() < 0.6 else int(rng.integers(0, len(b)))
        b[p] ^= int(rng.integers(1, 256))
        try:
            bc.decode(bytes(b), {}, w.size, elem_bytes=w.dtype.itemsize)
            decoded += 1
        except (ValueError, DecodeError):
            raised += 1
    assert raised > 0 and raised + decoded == 120
