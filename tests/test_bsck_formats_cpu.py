"""The BSCK format's tANS coder, fp8 exponent-pair mode and layout version 2,
pinned on the CPU (oracle/bs_oracle.c's decoder is the checker).

* A hand-built tANS blob: two symbols, and a table chosen so that its decode
  follows from the format alone: position p holds symbol p & 1 with nb = 1
  and newX = p with its low bit cleared, so every state emits its low bit and
  takes the next stream bit in its place. A state X0 in {0, 1} then decodes
  X0 & 1 at step 0 and its first stream bit at step 1, and must end at 0. With
  128 states (two per lane) every step reads one bit per state in chunk
  element order, so the expected words follow from the states and bits
  directly; reading MSB first, group-major instead of lane-major, or from the
  wrong end breaks it. The same blob in coder 2 carries X0 as 12-bit fields
  at the head of the stream, lane-major (state g of lane l at bit
  12 * (l * 2 + g)), and its planted mistakes are group-major or MSB-first
  fields.
* Round trips of the product encoder through the oracle for both coders and
  every plane mode, with the tANS table the blob stores equal to the oracle's
  own construction from the quantised frequencies.
* The layout-version-2 blobs the earlier encoder wrote
  (tests/golden/make_bsck_v2.py) decode to their sources.
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np
import pytest

import oracle
from bigsmall_amd.codecs import bf16_chunked as bc

GOLDEN = Path(__file__).resolve().parent / "golden"


def _bf16(x: np.ndarray) -> np.ndarray:
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _fields12(vals, msb_first: bool = False) -> np.ndarray:
    """12-bit fields as stream bits, LSB first (or each field reversed)."""
    bits = (np.asarray(vals, np.int64)[:, None] >> np.arange(12)) & 1
    return (bits[:, ::-1] if msb_first else bits).reshape(-1)


def hand_built_tans(seed: int = 0, coder: int = 1, head_order: str = "lane", msb_first: bool = False):
    """(blob, expected words) of the hand-built tANS blob described above:
    bf16 exact-value symbols 1.0 and 2.0, 128 states, 2 steps (256 elements).
    Coder 2 puts the states at the stream head in `head_order` ("lane": the
    format's; "group": a planted mistake), fields LSB first unless
    `msb_first`."""
    rng = np.random.default_rng(seed)
    lanes, steps, n = 128, 16, 256
    A, B = 0x3F80, 0x4000
    sym = rng.integers(0, 2, n)                        # element j's symbol index
    x0 = sym[:128]                                     # step 0: element l*2+g is state v = g*64 + l
    bits = np.concatenate([sym[128:], np.zeros(128, np.int64)])   # stream: step 1's symbols, then zeros
    head = b"BSCK" + bytes([3, 2, 0, 12]) + struct.pack("<QIHHI", n, steps, lanes, 2, 1) + bytes([coder, 0, 0, 0])
    syms = struct.pack("<II", A | (2048 << 16), B | (2048 << 16))
    stab = 48
    table = np.array([(p & ~1) | (1 << 12) | ((p & 1) << 16) for p in range(4096)], np.uint32).tobytes()
    ctab = stab + 4 * 4096
    off = ctab + 16
    states = np.zeros(128, np.uint32)
    for j in range(128):
        l, g = j // 2, j % 2
        states[g * 64 + l] = x0[j]
    if coder == 2:
        order = x0 if head_order == "lane" else states       # states[v] is group-major
        bits = np.concatenate([_fields12(order, msb_first), bits])
        body = np.packbits(bits.astype(np.uint8), bitorder="little").tobytes()
    else:
        body = states.tobytes() + np.packbits(bits.astype(np.uint8), bitorder="little").tobytes()
    blob = head + syms + b"\0" * (stab - 40) + table + struct.pack("<QII", off, bits.size, 0) + body
    blob += b"\0" * (max(off + 256 - len(blob), 0) + (-max(len(blob), off + 256)) % 256)
    want = np.where(sym == 0, A, B).astype(np.uint16)
    return blob, want


def test_hand_built_tans_blob():
    oracle.build()
    for coder in (1, 2):
        blob, want = hand_built_tans(coder=coder)
        assert len(blob) % 256 == 0 and blob[28] == coder
        assert oracle.chunk_decode(blob, want.size) == want.tobytes(), coder


def test_hand_built_tans_head_states_planted_mistakes():
    """Coder 2 with the head states group-major or MSB first changes the
    decode (or fails it); so does the blob cut to less than 256 bytes past
    its chunk's offset."""
    oracle.build()
    blob, want = hand_built_tans(2, coder=2)
    for kw in (dict(head_order="group"), dict(msb_first=True)):
        bad, _ = hand_built_tans(2, coder=2, **kw)
        assert bad != blob
        try:
            got = oracle.chunk_decode(bad, want.size)
        except oracle.OracleError:
            continue
        assert got != want.tobytes(), kw
    off = 48 + 4 * 4096 + 16
    assert len(blob) >= off + 256
    with pytest.raises(oracle.OracleError):
        oracle.chunk_decode(blob[:off + 240], want.size)


def test_hand_built_tans_planted_mistakes():
    """Flipping the stream's bit order, a state or a table entry each changes
    the decode (or fails it)."""
    blob, want = hand_built_tans(1)
    stab, off = 48, 48 + 4 * 4096 + 16
    bad = []
    b = bytearray(blob)                                # MSB-first stream bytes
    for i in range(off + 512, off + 512 + 32):
        b[i] = int(f"{b[i]:08b}"[::-1], 2)
    bad.append(bytes(b))
    b = bytearray(blob); b[off] ^= 1                   # state 0's first symbol
    bad.append(bytes(b))
    b = bytearray(blob); b[stab + 4 * 1 + 2] ^= 1      # position 1 (a state value in use) decodes the other symbol
    bad.append(bytes(b))
    for i, x in enumerate(bad):
        try:
            got = oracle.chunk_decode(x, want.size)
        except oracle.OracleError:
            continue
        assert got != want.tobytes(), i


def _inputs(rng):
    g = _bf16(rng.standard_normal(150_001) * 0.02)
    hz = _bf16(rng.standard_normal(90_001) * 0.02)
    hz[rng.permutation(hz.size)[: hz.size // 2]] = 0
    import torch
    f8 = torch.from_numpy(rng.standard_normal(80_000).astype(np.float32)).to(torch.float8_e4m3fn)
    yield "gauss", g, [-1, 1, 2]
    yield "studentt", _bf16(rng.standard_t(3, 70_000) * 0.02), [-1, 1]
    yield "halfzero", hz, [-1, 2, 1]
    yield "norms", _bf16(1.0 + rng.standard_normal(4096) * 0.01), [-1, 0]
    yield "uniform", rng.integers(0, 65536, 30_000).astype(np.uint16), [1]
    yield "fp8", f8.view(torch.uint8).numpy().copy(), [-1, 0, 3]
    yield "fp8_odd", f8.view(torch.uint8).numpy()[:12_345].copy(), [-1, 0]
    yield "one", np.array([0x3F80], np.uint16), [-1, 1]


@pytest.mark.parametrize("coder", [0, 1, 2])
@pytest.mark.parametrize("lanes", [64, 128, 256])
def test_round_trips_through_the_oracle(coder, lanes):
    oracle.build()
    rng = np.random.default_rng(lanes + coder)
    for name, w, modes in _inputs(rng):
        for mode in modes:
            blob = bc.encode_array(w, steps=32, mode=mode, lanes=lanes, coder=coder)
            assert blob[28] == coder and (mode < 0 or blob[6] == mode), (name, mode)
            assert oracle.chunk_decode(blob, w.size, w.dtype.itemsize) == w.tobytes(), (name, mode)
            if coder != 0:
                nsym = struct.unpack_from("<H", blob, 22)[0]
                freqs = [(struct.unpack_from("<I", blob, 32 + 4 * s)[0] >> 16) & 0x1FFF for s in range(nsym)]
                stab = (32 + 4 * nsym + 15) & ~15
                assert np.array_equal(np.frombuffer(blob, np.uint32, 4096, stab), oracle.tans_table(freqs)), name


def test_fp8_pairs_chosen_for_normal_fp8_and_byte_mode_for_odd_counts():
    import torch
    f8 = torch.randn(1 << 20, generator=torch.Generator().manual_seed(4)).to(torch.float8_e4m3fn)
    w = f8.view(torch.uint8).numpy()
    assert bc.encode_array(w, steps=128)[6] == 3          # within 2 % of byte symbols: pairs
    assert bc.encode_array(w[:-1], steps=128)[6] == 0     # odd count: bytes
    with pytest.raises(RuntimeError):
        bc.encode_array(w[:-1], steps=128, mode=3)


def test_tans_table_has_the_spread_and_state_ranges():
    """Closed-form properties of the oracle's table: every symbol owns exactly
    f positions, newX + 2^nb stays within the table, and the states a symbol
    leads to cover [0, 4096) once over its positions' bit ranges."""
    rng = np.random.default_rng(9)
    f = np.bincount(rng.integers(0, 20, 4096), minlength=20)
    f = f[f > 0].astype(np.uint32)
    f[0] += 4096 - f.sum()
    t = oracle.tans_table(f)
    sym, nb, nx = (t >> 16) & 0xFF, (t >> 12) & 15, t & 0xFFF
    assert np.array_equal(np.bincount(sym, minlength=len(f)), f)
    assert np.all(nx + (1 << nb) <= 4096) and np.all(nx % (1 << nb) == 0)
    for s in range(len(f)):
        cover = np.zeros(4096, np.int64)
        for p in np.flatnonzero(sym == s):
            cover[nx[p]:nx[p] + (1 << nb[p])] += 1
        assert np.all(cover == 1), s
    # position p holds the symbol of sorted slot p * 2563^-1 mod 4096
    inv = pow(2563, -1, 4096)
    cum = np.concatenate([[0], np.cumsum(f)])
    slot = (np.arange(4096) * inv) % 4096
    assert np.array_equal(sym, np.searchsorted(cum, slot, side="right") - 1)


def test_layout_version_2_golden_blobs():
    oracle.build()
    z = np.load(GOLDEN / "bsck_v2_vectors.npz")
    names = [k[4:] for k in z.files if k.startswith("src_")]
    assert len(names) >= 6
    for name in names:
        src, blob = z["src_" + name], z["blob_" + name].tobytes()
        assert blob[4] == 2
        assert oracle.chunk_decode(blob, src.size, src.dtype.itemsize) == src.tobytes(), name
        info = bc.info(blob)
        assert info.n == src.size and info.coder == 0
