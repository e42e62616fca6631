"""Pin the oracle (oracle/bs_oracle.c) before trusting it.

1. Golden vectors written from the reference's own pure-Python modules
   (tests/golden/make_golden.py): quantisers, rANS streams, and the exact blobs
   of bf16_parallel_v1 / bf16_se_tans / bf16_se_single_kernel.
2. Closed forms: a single-symbol stream is exactly the state L (b"\\x00\\x00\\x01\\x00");
   an empty tensor encodes to b"".
3. Planted mistakes: perturbed oracle inputs (a flipped blob byte, a wrong
   frequency) must change the result, so the checks above are not vacuous.
"""
from __future__ import annotations

import hashlib

import numpy as np
import pytest

import oracle


@pytest.fixture(scope="module", autouse=True)
def _built():
    oracle.build()


def _cases(golden, prefix):
    return sorted(k for k in golden if k.startswith(prefix))


def test_quantisers_match_reference(golden):
    n = 0
    for k in _cases(golden, "q"):
        if not k.endswith("_counts"):
            continue
        i = k[: -len("_counts")]
        c, M = golden[k], int(golden[f"{i}_M"][0])
        if f"{i}_ref_raises" in golden:
            with pytest.raises(oracle.OracleError):
                oracle.quantise_ref(c, M)
        else:
            assert np.array_equal(oracle.quantise_ref(c, M), golden[f"{i}_ref"]), i
        assert np.array_equal(oracle.quantise_sk(c, M), golden[f"{i}_sk"]), i
        n += 1
    assert n >= 8


def test_quantise_sums_and_floor():
    rng = np.random.default_rng(0)
    for _ in range(50):
        c = rng.integers(0, 50, 512) * (rng.random(512) < 0.3)
        if c.sum() == 0:
            continue
        f = oracle.quantise_ref(c, 4096)
        assert f.sum() == 4096
        assert np.all((f > 0) == (c > 0))
        g = oracle.quantise_sk(c, 4096)
        assert g.sum() == 4096 and np.all((g > 0) == (c > 0))


def test_rans_streams_match_reference(golden):
    for k in _cases(golden, "s"):
        if not k.endswith("_syms"):
            continue
        i = k[: -len("_syms")]
        syms, freqs, M = golden[k], golden[f"{i}_freqs"], int(golden[f"{i}_M"][0])
        blob = golden[f"{i}_blob"].tobytes()
        assert oracle.rans_encode(syms, freqs, M) == blob
        assert np.array_equal(oracle.rans_decode(blob, len(syms), freqs, M), syms)
        prec = M.bit_length() - 1
        assert np.array_equal(oracle.rans_decode_nb(blob, len(syms), freqs, prec), syms)


def test_single_symbol_stream_closed_form():
    f = np.zeros(128, np.uint32)
    f[9] = 1024
    blob = oracle.rans_encode(np.full(777, 9), f, 1024)
    assert blob == b"\x00\x00\x01\x00"
    assert np.all(oracle.rans_decode(blob, 777, f, 1024) == 9)
    assert oracle.rans_encode(np.zeros(0), f, 1024) == b"\x00\x00\x01\x00"


@pytest.mark.parametrize("codec", ["par1", "tans", "sk"])
def test_codec_blobs_match_reference(golden, codec):
    enc = {"par1": oracle.par1_encode, "tans": oracle.tans_encode, "sk": oracle.sk_encode}[codec]
    dec = {"par1": oracle.par1_decode, "tans": oracle.tans_decode, "sk": oracle.sk_decode}[codec]
    seen = 0
    for k in _cases(golden, codec + "_"):
        name = k[len(codec) + 1:]
        ns = None
        if codec == "par1":
            name, ns = name.rsplit("_N", 1)
            ns = int(ns)
        words = golden[f"in_{name}"]
        ref = golden[k].tobytes()
        mine = enc(words, ns) if ns else enc(words)
        assert mine == ref, f"{k}: oracle encoder differs from reference bytes"
        out = dec(ref, len(words))
        assert out == words.astype("<u2").tobytes(), f"{k}: decode is not lossless"
        seen += 1
    assert seen >= 7


def test_empty_and_clamped():
    assert oracle.par1_encode(np.zeros(0, np.uint16)) == b""
    assert oracle.par1_decode(b"", 0) == b""
    w = np.array([0x3F80, 0xBF80, 0x0001], np.uint16)
    blob = oracle.par1_encode(w, 128)               # N clamps to n (bf16_parallel.py:195)
    assert int.from_bytes(blob[8:10], "little") == 3
    assert oracle.par1_decode(blob, 3) == w.tobytes()


def test_planted_mistakes_are_caught(golden):
    words = golden["in_gauss"]
    ref = golden["par1_gauss_N64"].tobytes()
    good = hashlib.md5(words.tobytes()).hexdigest()
    bad = bytearray(ref)
    bad[len(bad) // 2] ^= 0x5A
    try:
        out = oracle.par1_decode(bytes(bad), len(words))
        assert hashlib.md5(out).hexdigest() != good
    except oracle.OracleError:
        pass
    # a wrong frequency table must not reproduce the reference stream
    syms, freqs, M = golden["s0_syms"], golden["s0_freqs"].copy(), int(golden["s0_M"][0])
    big = np.nonzero(freqs > 1)[0]
    small = [i for i in np.nonzero(freqs)[0] if i != big[0]]
    freqs[big[0]] -= 1
    freqs[small[0]] += 1
    assert oracle.rans_encode(syms, freqs, M) != golden["s0_blob"].tobytes()


def test_tans_and_sk_roundtrip_random():
    rng = np.random.default_rng(3)
    for n in [1, 2, 255, 10000]:
        x = (rng.standard_normal(n) * 0.02).astype(np.float32)
        w = (x.view(np.uint32) >> 16).astype(np.uint16)
        for enc, dec in [(oracle.tans_encode, oracle.tans_decode), (oracle.sk_encode, oracle.sk_decode),
                         (oracle.par1_encode, oracle.par1_decode)]:
            assert dec(enc(w), n) == w.tobytes()
