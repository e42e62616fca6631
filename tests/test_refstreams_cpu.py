"""CPU checks of the host side of the GPU decoders for the reference's formats
(bf16_parallel_v1, bf16_se_tans, bf16_se_single_kernel).

The host parses a blob into stream descriptors, bucket start tables and decode
tables (bigsmall_amd/codecs/_refstreams.py). Here plain-Python emulations of
the device kernels' semantics (refcodec_decode.hip: se_kernel + mant_kernel,
and the wave-serial path for one-stream formats) run on those descriptors, for every reference blob in the golden fixtures
(written by the reference's own encoders), and must give back the original
words. Malformed framing must raise ValueError.
"""
from __future__ import annotations

import numpy as np
import pytest

from bigsmall_amd.codecs import _refstreams as rs

L = 1 << 16


def _word(blob: bytes, off: int, i: int) -> int:
    return blob[off + 2 * i] | (blob[off + 2 * i + 1] << 8)


def _run(blob: bytes, s: rs.Stream, n: int, table, precision: int):
    """Decode n symbols of one stream with the kernels' loop; returns (symbols, end state, words used)."""
    n_eff = s.n_words + ((s.tail >> 16) & 1)
    x, pos, out = s.x0, 0, []
    mask = (1 << precision) - 1
    for _ in range(n):
        f, bias, sym = table(x & mask)
        x = f * (x >> precision) + bias
        while x < L and pos < n_eff:
            v = _word(blob, s.words_off, pos) if pos < s.n_words else (s.tail & 0xFFFF)
            x = ((x << 16) | v) & 0xFFFFFFFF
            pos += 1
        out.append(sym)
    return out, x, pos, n_eff


def emulate(plan: rs.RefPlan, blob: bytes) -> np.ndarray:
    se_t = rs.decode_table_se(plan.se_freqs)
    mts = [rs.decode_table_mant(f) for f in plan.mant_freqs]
    out = np.zeros(plan.n, np.uint16)
    perm = np.full(plan.n, -1, np.int64)
    for (s, first, stride, n), bs in zip(plan.se_streams, plan.bstart):
        syms, x, pos, n_eff = _run(blob, s, n, lambda sl: (int(se_t[sl, 0]) & 0x1FFF, int(se_t[sl, 0]) >> 13,
                                                           int(se_t[sl, 1])), 12)
        assert x == L and pos == n_eff
        cur = bs[:256].astype(np.int64).copy()
        for i, sym in enumerate(syms):
            e = sym & 0xFF
            idx = first + i * stride
            out[idx] = ((sym >> 8) & 1) << 15 | e << 7
            perm[cur[e]] = idx
            cur[e] += 1
        assert np.array_equal(cur, bs[1:].astype(np.int64))
    for s, pb, n, t in plan.buckets:
        tbl = mts[t]
        syms, x, pos, n_eff = _run(blob, s, n, lambda sl: (int(tbl[sl]) & 0x7FF, (int(tbl[sl]) >> 11) & 0x3FF,
                                                           int(tbl[sl]) >> 21), 10)
        assert x == L and pos == n_eff
        for r, m in enumerate(syms):
            out[perm[pb + r]] |= m
    return out


def emulate_serial(plan: rs.RefPlan, blob: bytes, tile: int = 256) -> np.ndarray:
    """The wave-serial path (refcodec_decode.hip: serial_kernel, hist_kernel,
    scan_kernel, place_kernel): each SE chain writes sign<<15 | exp<<7 at its
    elements first + i*stride, each mantissa chain writes its bucket in bucket
    order, then per stream: tile exponent histograms over the stream's symbol
    index, a scan over its tiles per exponent from bstart, and per-64-symbol
    ranks place every element's mantissa."""
    se_t = rs.decode_table_se(plan.se_freqs)
    n = plan.n
    out = np.zeros(n, np.uint16)
    for s, first, stride, ns in plan.se_streams:
        syms, x, pos, n_eff = _run(blob, s, ns, lambda sl: (int(se_t[sl, 0]) & 0x1FFF, int(se_t[sl, 0]) >> 13,
                                                            int(se_t[sl, 1])), 12)
        assert x == L and pos == n_eff
        syms = np.asarray(syms, np.uint32)
        out[first + stride * np.arange(ns)] = (((syms >> 8) & 1) << 15) | ((syms & 0xFF) << 7)
    mant = np.zeros(n, np.uint8)
    for bs_, pb, nb, t in plan.buckets:
        tbl = rs.decode_table_mant(plan.mant_freqs[t])
        m, x, pos, n_eff = _run(blob, bs_, nb, lambda sl: (int(tbl[sl]) & 0x7FF, (int(tbl[sl]) >> 11) & 0x3FF,
                                                           int(tbl[sl]) >> 21), 10)
        assert x == L and pos == n_eff
        mant[pb:pb + nb] = m
    for (s, first, stride, ns), bstart in zip(plan.se_streams, plan.bstart):
        elems = first + stride * np.arange(ns)
        e = (out[elems] >> 7) & 0xFF
        tiles = (ns + tile - 1) // tile
        hist = np.zeros((tiles, 256), np.int64)
        for t in range(tiles):
            hist[t] = np.bincount(e[t * tile:(t + 1) * tile], minlength=256)
        bstart = bstart.astype(np.int64)
        firsts = bstart[:256] + np.concatenate([np.zeros((1, 256), np.int64), np.cumsum(hist, 0)[:-1]])
        assert np.array_equal(bstart[:256] + hist.sum(0), bstart[1:])
        for t in range(tiles):
            cnt = firsts[t].copy()
            for k0 in range(t * tile, min(ns, (t + 1) * tile), 64):
                ch = e[k0:min(ns, k0 + 64)]
                for lane, ev in enumerate(ch):
                    rank = int(np.count_nonzero(ch[:lane] == ev))
                    out[elems[k0 + lane]] |= mant[cnt[ev] + rank]
                for ev in np.unique(ch):
                    cnt[ev] += int(np.count_nonzero(ch == ev))
    return out


@pytest.mark.parametrize("codec,prefix", [("bf16_parallel_v1", "par1_"), ("bf16_se_tans", "tans_"),
                                          ("bf16_se_single_kernel", "sk_")])
def test_serial_path_decodes_reference_blobs(golden, codec, prefix):
    seen = 0
    for k in sorted(golden):
        if not k.startswith(prefix):
            continue
        name = k[len(prefix):].rsplit("_N", 1)[0] if prefix == "par1_" else k[len(prefix):]
        words = golden[f"in_{name}"].astype(np.uint16)
        if words.size > 40000 or words.size == 0:
            continue
        blob = golden[k].tobytes()
        assert np.array_equal(emulate_serial(rs.PARSERS[codec](blob, words.size), blob), words), k
        seen += 1
    assert seen >= 5


@pytest.mark.parametrize("codec,prefix", [("bf16_parallel_v1", "par1_"), ("bf16_se_tans", "tans_"),
                                          ("bf16_se_single_kernel", "sk_")])
def test_host_plans_decode_reference_blobs(golden, codec, prefix):
    seen = 0
    for k in sorted(golden):
        if not k.startswith(prefix):
            continue
        name = k[len(prefix):].rsplit("_N", 1)[0] if prefix == "par1_" else k[len(prefix):]
        words = golden[f"in_{name}"].astype(np.uint16)
        if words.size > 40000:
            continue                       # the pure-Python emulation is slow; GPU tests cover these
        blob = golden[k].tobytes()
        plan = rs.PARSERS[codec](blob, words.size)
        assert np.array_equal(emulate(plan, blob), words), k
        seen += 1
    assert seen >= 5


def test_tables_are_exact_inverses():
    rng = np.random.default_rng(0)
    f = np.zeros(512, np.int64)
    f[rng.choice(512, 30, replace=False)] = 1
    f[np.nonzero(f)[0][0]] += 4096 - f.sum()
    t = rs.decode_table_se(f)
    cum = np.concatenate([[0], np.cumsum(f)[:-1]])
    for slot in range(0, 4096, 17):
        sym = t[slot, 1]
        assert cum[sym] <= slot < cum[sym] + f[sym]
        assert t[slot, 0] & 0x1FFF == f[sym] and t[slot, 0] >> 13 == slot - cum[sym]


def test_malformed_blobs_raise(golden):
    blob = golden["par1_gauss_N64"].tobytes()
    n = golden["in_gauss"].size
    with pytest.raises(ValueError):
        rs.parse_parallel(blob, n + 1)              # wrong count
    with pytest.raises(ValueError):
        rs.parse_parallel(blob[: len(blob) // 2], n)  # truncated
    bad = bytearray(blob)
    bad[0:4] = b"PAR2"
    with pytest.raises(ValueError):
        rs.parse_parallel(bytes(bad), n)
    tb = golden["tans_gauss"].tobytes()
    with pytest.raises(ValueError):
        rs.parse_tans(tb[:100], n)
    sk = golden["sk_gauss"].tobytes()
    with pytest.raises(ValueError):
        rs.parse_single_kernel(sk[:-3], n)


@pytest.mark.parametrize("groups,lens", [
    ([32] * 7, [131072, 32768, 32768, 131072, 458752, 458752, 458752]),   # the 8B layer in bf16_parallel_v1
    ([1] * 7, [7, 6, 5, 4, 3, 2, 1]),                                     # the same layer in bf16_se_tans
    ([32] * 20, list(range(20))),
    ([3, 1, 1, 1, 1, 1, 1, 1, 1, 1], [9, 8, 7, 6, 5, 4, 3, 2, 1, 0]),
    ([5, 40, 2, 2, 9, 33, 1, 1, 1, 17, 8], [10, 99, 3, 3, 20, 70, 1, 2, 1, 50, 9]),
])
def test_xcd_bins_layout(groups, lens):
    """Each task's SE groups sit inside one of the 8 bins of C groups, no two
    overlap, the task array ascends, the first task of each bin has the
    longest chains in it, and the longest eight tasks lead eight bins."""
    C, order, begin, first = rs.xcd_bins(groups, lens)
    assert sorted(order) == list(range(len(groups)))
    assert [begin[i] for i in order] == sorted(begin[i] for i in order)
    used = set()
    for i in order:
        lo, hi = begin[i], begin[i] + groups[i]
        assert lo // C == (hi - 1) // C and hi <= rs.XCD_BINS * C, (i, lo, hi, C)
        span = set(range(lo, hi))
        assert not (span & used)
        used |= span
    for j in range(rs.XCD_BINS):
        members = [i for i in order if begin[i] // C == j]
        if members:
            assert first[members[0]] and not any(first[i] for i in members[1:])
            assert lens[members[0]] == max(lens[i] for i in members)
    longest = sorted(range(len(groups)), key=lambda i: (-lens[i], -groups[i], i))[:rs.XCD_BINS]
    assert all(first[i] for i in longest)
    assert C >= max(groups) and rs.XCD_BINS * C >= sum(groups)


def test_xcd_bins_one_task_spreads():
    assert rs.xcd_bins([32], [131072]) == (4, [0], {0: 0}, {0: True})
    assert rs.xcd_bins([1], [5]) == (1, [0], {0: 0}, {0: True})
