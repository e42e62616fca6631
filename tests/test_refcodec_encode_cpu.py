"""The library's host encoders of the reference's formats (bs_refcodec_encode,
bigsmall_amd/csrc/refcodec_encode.cpp) on the CPU.

1. Byte-identical to the blobs the reference's own encoders wrote for the
   golden inputs (tests/golden/ref_vectors.npz): bf16_parallel_v1 at N in
   {1, 3, 32, 64, 128}, bf16_se_tans, bf16_se_single_kernel.
2. Byte-identical to the oracle's encoders (which the same golden blobs pin)
   on larger and adversarial inputs, and decoded back by the oracle's decoders.
3. Edge cases: empty input -> b"", odd byte counts raise, N clamps to n.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from bigsmall_amd.codecs import _refstreams, bf16_parallel, bf16_tans, single_kernel


@pytest.fixture(scope="module", autouse=True)
def _built():
    oracle.build()


def _bf16(x: np.ndarray) -> np.ndarray:
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def test_golden_blobs_byte_identical(golden):
    n = 0
    for k in sorted(golden):
        if k.startswith("par1_"):
            name, ns = k[len("par1_"):].rsplit("_N", 1)
            w = golden[f"in_{name}"].astype("<u2")
            blob, extras = bf16_parallel.encode(w.tobytes(), n_streams=int(ns))
            assert extras == {"n_streams": max(1, min(int(ns), w.size))}
        elif k.startswith("tans_"):
            w = golden[f"in_{k[5:]}"].astype("<u2")
            blob, _ = bf16_tans.encode(w.tobytes())
        elif k.startswith("sk_"):
            w = golden[f"in_{k[3:]}"].astype("<u2")
            blob, _ = single_kernel.encode(w.tobytes())
        else:
            continue
        assert blob == golden[k].tobytes(), k
        n += 1
    assert n >= 28


def _inputs():
    rng = np.random.default_rng(17)
    yield "gauss", _bf16(rng.standard_normal(300_001) * 0.02)
    yield "studentt", _bf16(rng.standard_t(3, 200_000) * 0.02 / np.sqrt(3))
    hz = _bf16(rng.standard_normal(150_000) * 0.02)
    hz[rng.permutation(hz.size)[: hz.size // 2]] = 0
    yield "halfzero", hz
    yield "uniform", rng.integers(0, 65536, 100_000).astype(np.uint16)
    yield "constant", np.full(70_000, 0x3F80, np.uint16)
    yield "one", np.array([0xBF80], np.uint16)
    yield "two_exps", np.array([0x0001, 0x7F7F] * 999, np.uint16)


@pytest.mark.parametrize("codec", ["bf16_parallel_v1", "bf16_se_tans", "bf16_se_single_kernel"])
def test_matches_oracle_and_round_trips(codec):
    enc, dec = {"bf16_parallel_v1": (oracle.par1_encode, oracle.par1_decode),
                "bf16_se_tans": (oracle.tans_encode, oracle.tans_decode),
                "bf16_se_single_kernel": (oracle.sk_encode, oracle.sk_decode)}[codec]
    for name, w in _inputs():
        for threads in (1, 5):
            blob = _refstreams.encode_host(codec, w.tobytes(), threads=threads)
            assert blob == enc(w), (codec, name, threads)
        assert dec(blob, w.size) == w.tobytes(), (codec, name)


def test_parallel_stream_counts_and_clamp():
    w = _bf16(np.random.default_rng(3).standard_normal(5_000) * 0.02)
    # N = max(1, min(n_streams, n)) (bf16_parallel.py:195): 0, negative and
    # oversized counts write the clamped count's blob, as the reference does
    for ns in (-3, 0, 1, 2, 7, 128, 4999, 5000, 5001, 65535, 100_000):
        blob, extras = bf16_parallel.encode(w.tobytes(), n_streams=ns)
        assert blob == oracle.par1_encode(w, max(1, min(ns, w.size))), ns
        assert extras["n_streams"] == max(1, min(ns, w.size))
    # a clamped N above 65535 does not fit the header's u16 (struct '<H' raises in the reference)
    big = _bf16(np.random.default_rng(4).standard_normal(70_000) * 0.02)
    with pytest.raises(RuntimeError):
        bf16_parallel.encode(big.tobytes(), n_streams=66_000)


def test_empty_and_odd_inputs():
    assert bf16_parallel.encode(b"") == (b"", {"n_streams": 128})
    assert bf16_tans.encode(b"") == (b"", {})
    assert single_kernel.encode(b"") == (b"", {})
    for enc in (bf16_parallel.encode, bf16_tans.encode, single_kernel.encode):
        with pytest.raises(ValueError):
            enc(b"\x00\x01\x02")
