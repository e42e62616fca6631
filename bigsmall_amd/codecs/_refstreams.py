"""Host side of the GPU decoders for the reference's rANS-family bf16 formats.

The reference decodes these formats on the CPU, symbol by symbol:
    bf16_parallel_v1       bigsmall/codecs/bf16_parallel.py:262-352 (streams: rans.py:165-207)
    bf16_se_tans           bigsmall/codecs/bf16_tans.py:121-167 (streams: numba_rans.py:168-192)
    bf16_se_single_kernel  bigsmall/codecs/single_kernel.py:431-580
Here the host only walks the blob's framing (a few hundred header fields)
into stream descriptors and decode tables; every symbol is decoded by
`bs_refcodec_decode` (bigsmall_amd/csrc/refcodec_decode.hip) on the GPU.

Each format codes a bf16 word as a 9-bit sign+exponent symbol (M = 4096)
plus its 7-bit mantissa in a per-exponent "bucket" (M = 1024); buckets hold
the mantissas of the elements sharing an exponent in element order. The
decoder places bucket (stream, e) at perm[bstart[stream][e]:...], where
bstart is the prefix sum of the header's bucket sizes in ascending exponent
order, which is where the reference's stable argsort puts them.

Deviation on malformed input only: the reference raises on some framing
errors and silently returns garbage on others (wrong counts, corrupt words);
this decoder raises ValueError for framing errors and reports corrupt streams
through the device status word (DecodeError).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

from .. import _native

M_SE, M_MANT = 4096, 1024
SERIAL_MIN_ELEMENTS = 1 << 16   # from here on a wavefront per chain beats a lane per chain
SE_ALPHABET, MANT_ALPHABET = 512, 128

SE_STREAM_DTYPE = np.dtype([("words", "<u8"), ("x0", "<u4"), ("n_words", "<u4"), ("tail", "<u4"), ("n", "<u4"),
                            ("first", "<u8"), ("stride", "<u4"), ("reserved", "<u4")])
MANT_BUCKET_DTYPE = np.dtype([("words", "<u8"), ("x0", "<u4"), ("n_words", "<u4"), ("tail", "<u4"), ("n", "<u4"),
                              ("perm_begin", "<u8"), ("table", "<u4"), ("reserved", "<u4")])
REF_TASK_DTYPE = np.dtype([("streams", "<u8"), ("se_table", "<u8"), ("bstart", "<u8"), ("buckets", "<u8"),
                           ("mant_tables", "<u8"), ("out", "<u8"), ("n_out", "<u8"), ("work_offset", "<u8"),
                           ("n_streams", "<u4"), ("n_buckets", "<u4"), ("n_tables", "<u4"), ("se_group_begin", "<u4"),
                           ("tile_begin", "<u4"), ("stream_begin", "<u4"), ("mant_group_begin", "<u4"),
                           ("flags", "<u4")])
# bs_ref_task.flags (include/bigsmall_hip.h)
FLAG_SE_SCALAR, FLAG_MANT_SCALAR = 1, 2
assert SE_STREAM_DTYPE.itemsize == 40 and MANT_BUCKET_DTYPE.itemsize == 40 and REF_TASK_DTYPE.itemsize == 96


class _Reader:
    """Little-endian cursor over a blob; short reads raise ValueError."""

    def __init__(self, blob: bytes, pos: int = 0, end: int | None = None, what: str = "blob"):
        self.b, self.pos, self.end, self.what = blob, pos, len(blob) if end is None else end, what

    def take(self, n: int) -> int:
        if n < 0 or self.pos + n > self.end:
            raise ValueError(f"{self.what}: truncated (need {n} bytes at {self.pos}, have {self.end - self.pos})")
        p = self.pos
        self.pos += n
        return p

    def u8(self) -> int:
        return self.b[self.take(1)]

    def u16(self) -> int:
        return struct.unpack_from("<H", self.b, self.take(2))[0]

    def u32(self) -> int:
        return struct.unpack_from("<I", self.b, self.take(4))[0]

    def arr(self, dtype: str, count: int) -> np.ndarray:
        size = np.dtype(dtype).itemsize * count
        return np.frombuffer(self.b, dtype=dtype, count=count, offset=self.take(size)).copy()


@dataclass
class Stream:
    """One rANS stream: initial state, word array (blob offset), optional tail word."""
    x0: int
    words_off: int
    n_words: int
    tail: int = 0          # bit 16 set: one more word with value tail & 0xFFFF


def inline_stream(blob: bytes, off: int, length: int, tail_is_byte: bool, what: str) -> Stream:
    """[u32 x0][u16 words...] framing of rans.encode_stream / numba_rans.encode_stream.

    An odd trailing byte is one more word: the reference's rans.decode_stream
    shifts in zero for it (rans.py:196-203); numba_rans.decode_stream pads the
    blob to even length, so the word is the byte itself (numba_rans.py:209-210)."""
    if length < 4:
        raise ValueError(f"{what}: rANS stream too short for its state ({length} bytes)")
    x0 = struct.unpack_from("<I", blob, off)[0]
    body = length - 4
    tail = 0
    if body % 2:
        tail = 0x10000 | (blob[off + length - 1] if tail_is_byte else 0)
    return Stream(x0, off + 4, body // 2, tail)


def decode_table_se(freqs: np.ndarray) -> np.ndarray:
    """4096 x {f | (slot - cf) << 13, symbol} for a 512-symbol table summing to 4096."""
    freqs = np.asarray(freqs, dtype=np.int64)
    if freqs.sum() != M_SE:
        raise ValueError(f"sign/exponent frequencies sum to {int(freqs.sum())}, expected {M_SE}")
    sym = np.repeat(np.arange(len(freqs), dtype=np.int64), freqs)
    cum = np.concatenate([[0], np.cumsum(freqs)[:-1]])
    slot = np.arange(M_SE, dtype=np.int64)
    out = np.empty((M_SE, 2), np.uint32)
    out[:, 0] = (freqs[sym] | ((slot - cum[sym]) << 13)).astype(np.uint32)
    out[:, 1] = sym.astype(np.uint32)
    return out


def decode_table_se_scalar(freqs: np.ndarray):
    """The SE table's 4-byte form for a tensor with at most 256 live symbols,
    none of frequency 4096 (else None): 4096 x {index | f << 8 | (slot - cf)
    << 20} and the 256 output words (sign << 15 | exponent << 7) of the
    indexed live symbols, as one uint32 array of 4096 + 256 entries."""
    freqs = np.asarray(freqs, dtype=np.int64)
    live = np.flatnonzero(freqs)
    if len(live) > 256 or freqs.max() >= M_SE:
        return None
    index = np.zeros(len(freqs), np.int64)
    index[live] = np.arange(len(live))
    sym = np.repeat(np.arange(len(freqs), dtype=np.int64), freqs)
    cum = np.concatenate([[0], np.cumsum(freqs)[:-1]])
    slot = np.arange(M_SE, dtype=np.int64)
    packed = (index[sym] | (freqs[sym] << 8) | ((slot - cum[sym]) << 20)).astype(np.uint32)
    words = np.zeros(256, np.uint32)
    words[: len(live)] = (((live >> 8) & 1) << 15) | ((live & 0xFF) << 7)
    return np.concatenate([packed, words])


def decode_table_mant(freqs: np.ndarray) -> np.ndarray:
    """1024 x (f | (slot - cf) << 11 | symbol << 21) for a 128-symbol table summing to 1024."""
    freqs = np.asarray(freqs, dtype=np.int64)
    if freqs.sum() != M_MANT:
        raise ValueError(f"mantissa frequencies sum to {int(freqs.sum())}, expected {M_MANT}")
    sym = np.repeat(np.arange(len(freqs), dtype=np.int64), freqs)
    cum = np.concatenate([[0], np.cumsum(freqs)[:-1]])
    slot = np.arange(M_MANT, dtype=np.int64)
    return (freqs[sym] | ((slot - cum[sym]) << 11) | (sym << 21)).astype(np.uint32)


@dataclass
class RefPlan:
    """A parsed blob: everything bs_refcodec_decode needs, with blob offsets."""
    n: int
    se_freqs: np.ndarray
    se_streams: list = field(default_factory=list)      # (Stream, first, stride, n)
    bstart: list = field(default_factory=list)          # per SE stream: 257 perm indices
    buckets: list = field(default_factory=list)         # (Stream, perm_begin, n, table)
    mant_freqs: list = field(default_factory=list)      # per table: 128 freqs


def _bucket_starts(base: int, sizes: dict[int, int], total: int, what: str) -> np.ndarray:
    """perm index of each exponent's bucket (ascending exponent order)."""
    counts = np.zeros(256, np.int64)
    for e, c in sizes.items():
        if not 0 <= e < 256:
            raise ValueError(f"{what}: exponent {e} out of range")
        counts[e] += c
    if counts.sum() != total:
        raise ValueError(f"{what}: bucket sizes sum to {int(counts.sum())}, expected {total}")
    bs = np.zeros(257, np.int64)
    bs[1:] = np.cumsum(counts)
    return (bs + base).astype(np.uint32)


def parse_parallel(blob: bytes, n_weights: int) -> RefPlan:
    """bf16_parallel_v1 framing (bigsmall/codecs/bf16_parallel.py:106-183, 186-259)."""
    r = _Reader(blob, what="bf16_parallel")
    p = r.take(4)
    if bytes(blob[p:p + 4]) != b"PAR1":
        raise ValueError(f"bf16_parallel: bad magic {bytes(blob[p:p + 4])!r}")
    n = r.u32()
    n_streams = r.u16()
    p_se, p_m = r.u16(), r.u16()
    if p_se != 12 or p_m != 10:
        raise ValueError(f"bf16_parallel: precision mismatch (header SE={p_se} M={p_m} vs codec SE=12 M=10)")
    if n != n_weights:
        raise ValueError(f"bf16_parallel: weight count mismatch ({n} vs {n_weights})")
    n_se_nz = r.u16()
    se_idx = r.arr("<u2", n_se_nz)
    se_f = r.arr("<u4", n_se_nz)
    se_freqs = np.zeros(SE_ALPHABET, np.uint32)
    if len(se_idx) and se_idx.max() >= SE_ALPHABET:
        raise ValueError("bf16_parallel: sign/exponent symbol out of range")
    se_freqs[se_idx] = se_f
    n_exps = r.u32()
    exps = r.arr("<u2", n_exps)
    table_of: dict[int, int] = {}
    plan = RefPlan(n=n, se_freqs=se_freqs)
    for ev in exps:
        k = r.u8()
        idx = r.arr("<u1", k)
        f = r.arr("<u4", k)
        if len(idx) and idx.max() >= MANT_ALPHABET:
            raise ValueError("bf16_parallel: mantissa symbol out of range")
        mf = np.zeros(MANT_ALPHABET, np.uint32)
        mf[idx] = f
        table_of[int(ev)] = len(plan.mant_freqs)
        plan.mant_freqs.append(mf)
    if n_streams == 0:
        raise ValueError("bf16_parallel: zero streams")
    offs = r.arr("<u4", n_streams + 1)
    payload = r.pos
    base = 0
    for k in range(n_streams):
        nk = (n - 1 - k) // n_streams + 1 if k < n else 0
        if nk == 0:
            plan.bstart.append(None)
            continue
        lo, hi = payload + int(offs[k]), payload + int(offs[k + 1])
        if not payload <= lo <= hi <= len(blob):
            raise ValueError(f"bf16_parallel: stream {k} offsets out of range")
        s = _Reader(blob, lo, hi, what=f"bf16_parallel stream {k}")
        se_len = s.u32()
        se = inline_stream(blob, s.take(se_len), se_len, tail_is_byte=False, what=f"bf16_parallel stream {k}")
        plan.se_streams.append((se, k, n_streams, nk))
        m = s.u32()
        sexps = s.arr("<u2", m)
        sizes: dict[int, int] = {}
        bucket_meta = []
        for ev in sexps:
            count, blen = s.u32(), s.u32()
            mb = inline_stream(blob, s.take(blen), blen, tail_is_byte=False, what=f"bf16_parallel stream {k}")
            if int(ev) not in table_of:
                raise ValueError(f"bf16_parallel: stream {k} uses exponent {int(ev)} without a mantissa table")
            if int(ev) in sizes:
                raise ValueError(f"bf16_parallel: stream {k} lists exponent {int(ev)} twice")
            sizes[int(ev)] = count
            bucket_meta.append((mb, int(ev), count))
        bs = _bucket_starts(base, sizes, nk, f"bf16_parallel stream {k}")
        plan.bstart.append(bs)
        for mb, ev, count in bucket_meta:
            plan.buckets.append((mb, int(bs[ev]), count, table_of[ev]))
        base += nk
    plan.bstart = [b for b in plan.bstart if b is not None]
    return plan


def parse_tans(blob: bytes, n_weights: int) -> RefPlan:
    """bf16_se_tans framing (bigsmall/codecs/bf16_tans.py:68-167)."""
    r = _Reader(blob, what="bf16_se_tans")
    n = r.u32()
    if n != n_weights:
        raise ValueError(f"bf16_se_tans: count mismatch ({n} vs {n_weights})")
    n_se_nz = r.u16()
    se_idx = r.arr("<u2", n_se_nz)
    se_f = r.arr("<u4", n_se_nz)
    if len(se_idx) and se_idx.max() >= SE_ALPHABET:
        raise ValueError("bf16_se_tans: sign/exponent symbol out of range")
    se_freqs = np.zeros(SE_ALPHABET, np.uint32)
    se_freqs[se_idx] = se_f
    plan = RefPlan(n=n, se_freqs=se_freqs)
    se_len = r.u32()
    plan.se_streams.append((inline_stream(blob, r.take(se_len), se_len, True, "bf16_se_tans"), 0, 1, n))
    m_len = r.u32()
    m = _Reader(blob, r.take(m_len), r.pos, what="bf16_se_tans mantissa section")
    n_exps = m.u32()
    exps = m.arr("<u2", n_exps)
    sizes: dict[int, int] = {}
    meta = []
    for ev in exps:
        nb, n_nz = m.u32(), m.u8()
        idx = m.arr("<u1", n_nz)
        f = m.arr("<u4", n_nz)
        if len(idx) and idx.max() >= MANT_ALPHABET:
            raise ValueError("bf16_se_tans: mantissa symbol out of range")
        cw_len = m.u32()
        cw = inline_stream(blob, m.take(cw_len), cw_len, True, "bf16_se_tans bucket")
        if int(ev) in sizes:
            raise ValueError(f"bf16_se_tans: exponent {int(ev)} listed twice")
        sizes[int(ev)] = nb
        mf = np.zeros(MANT_ALPHABET, np.uint32)
        mf[idx] = f
        meta.append((cw, int(ev), nb, len(plan.mant_freqs)))
        plan.mant_freqs.append(mf)
    bs = _bucket_starts(0, sizes, n, "bf16_se_tans")
    plan.bstart.append(bs)
    plan.buckets = [(cw, int(bs[ev]), nb, t) for cw, ev, nb, t in meta]
    return plan


def parse_single_kernel(blob: bytes, n_weights: int) -> RefPlan:
    """bf16_se_single_kernel framing (bigsmall/codecs/single_kernel.py:303-321, 431-580)."""
    r = _Reader(blob, what="bf16_se_single_kernel")
    n = r.u32()
    if n != n_weights:
        raise ValueError(f"bf16_se_single_kernel: count mismatch ({n} vs {n_weights})")
    n_se_nz = r.u16()
    se_idx = r.arr("<u2", n_se_nz)
    se_f = r.arr("<u4", n_se_nz)
    if len(se_idx) and se_idx.max() >= SE_ALPHABET:
        raise ValueError("bf16_se_single_kernel: sign/exponent symbol out of range")
    se_freqs = np.zeros(SE_ALPHABET, np.uint32)
    se_freqs[se_idx] = se_f
    plan = RefPlan(n=n, se_freqs=se_freqs)
    x0, nw = r.u32(), r.u32()
    plan.se_streams.append((Stream(x0, r.take(2 * nw), nw), 0, 1, n))
    n_exps = r.u32()
    sizes: dict[int, int] = {}
    meta = []
    for _ in range(n_exps):
        ev, k = r.u16(), r.u8()
        idx = r.arr("<u1", k)
        f = r.arr("<u4", k)
        if len(idx) and idx.max() >= MANT_ALPHABET:
            raise ValueError("bf16_se_single_kernel: mantissa symbol out of range")
        mx0, bsize, mnw = r.u32(), r.u32(), r.u32()
        ms = Stream(mx0, r.take(2 * mnw), mnw)
        if ev in sizes:
            raise ValueError(f"bf16_se_single_kernel: exponent {ev} listed twice")
        sizes[ev] = bsize
        mf = np.zeros(MANT_ALPHABET, np.uint32)
        mf[idx] = f
        meta.append((ms, ev, bsize, len(plan.mant_freqs)))
        plan.mant_freqs.append(mf)
    bs = _bucket_starts(0, sizes, n, "bf16_se_single_kernel")
    plan.bstart.append(bs)
    plan.buckets = [(ms, int(bs[ev]), nb, t) for ms, ev, nb, t in meta]
    return plan


PARSERS = {"bf16_parallel_v1": parse_parallel, "bf16_se_tans": parse_tans,
           "bf16_se_single_kernel": parse_single_kernel}


def _plan_arrays(plan: RefPlan, blob_ptr: int) -> list[np.ndarray]:
    """The device arrays of one parsed blob, as host bytes: SE stream
    descriptors, SE decode table, bucket starts, bucket descriptors, mantissa
    decode tables."""
    se = np.zeros(len(plan.se_streams), SE_STREAM_DTYPE)
    for i, (s, first, stride, n) in enumerate(plan.se_streams):
        se[i] = (blob_ptr + s.words_off, s.x0, s.n_words, s.tail, n, first, stride, 0)
    # buckets longest first: the wave-serial kernel decodes them in groups of
    # four wavefronts, and a group holds its slot until its longest bucket ends
    # (every bucket carries its own output position, so the order is free)
    mb = np.zeros(len(plan.buckets), MANT_BUCKET_DTYPE)
    order = sorted(range(len(plan.buckets)), key=lambda i: -plan.buckets[i][2])
    for i, j in enumerate(order):
        s, pb, n, t = plan.buckets[j]
        mb[i] = (blob_ptr + s.words_off, s.x0, s.n_words, s.tail, n, pb, t, 0)
    tables = (np.stack([decode_table_mant(f) for f in plan.mant_freqs]) if plan.mant_freqs
              else np.zeros((1, M_MANT), np.uint32))
    se_table = decode_table_se(plan.se_freqs).reshape(-1)
    scalar = decode_table_se_scalar(plan.se_freqs)
    if scalar is not None:                  # the table's 4-byte form follows its pairs (BS_REF_FLAG_SE_SCALAR)
        se_table = np.concatenate([se_table, scalar])
    return [se.view(np.uint8), se_table.view(np.uint8),
            np.stack(plan.bstart).reshape(-1).view(np.uint8) if plan.bstart else np.zeros(0, np.uint8),
            mb.view(np.uint8), tables.reshape(-1).view(np.uint8)]


def _layout(arrays: list[np.ndarray]) -> tuple[int, list[int]]:
    """Offsets of byte arrays placed one after another on 256-byte boundaries."""
    offs, pos = [], 0
    for h in arrays:
        pos = (pos + 255) & ~255
        offs.append(pos)
        pos += h.nbytes
    return max(pos, 1), offs


def _pack(arrays: list[np.ndarray]) -> tuple[np.ndarray, list[int]]:
    """Concatenate byte arrays at 256-byte offsets; returns (buffer, offsets)."""
    size, offs = _layout(arrays)
    buf = np.zeros(size, np.uint8)
    for h, o in zip(arrays, offs):
        buf[o:o + h.nbytes] = h
    return buf, offs


def serial_ok(plan: RefPlan) -> bool:
    """The wave-serial path applies: a tensor of SERIAL_MIN_ELEMENTS or more
    whose streams each hold at most ceil(n / streams) symbols (every blob the
    reference's encoders write; a smaller tensor decodes as fast with one lane
    per chain)."""
    max_len = max((n for _, _, _, n in plan.se_streams), default=0)
    return plan.n >= SERIAL_MIN_ELEMENTS and len(plan.se_streams) > 0 and max_len <= -(-plan.n // len(plan.se_streams))


XCD_BINS = 8      # the chain kernel deals SE-group slot p to XCD p % 8 (round-robin dispatch)


def xcd_bins(groups: list, chain_len: list, n_bins: int = XCD_BINS) -> tuple:
    """Lay the tasks' SE groups out in n_bins equal bins of the SE part of the
    chain grid, bin j being what XCD j decodes (bs_refcodec_decode_serial_batch
    deals logical group (p % 8) * C + p / 8 to slot p of a grid of 8C): each
    task's groups stay in one bin, each task goes to the emptiest bin (ties
    to the lower bin), and C is the smallest capacity for which every task
    fits. Up to n_bins tasks each get a bin of their own in the caller's
    order; more are placed longest chains first, so the longest lead the
    bins. Returns (C, order, begin, first): the tasks in grid order, each
    task's se_group_begin, and whether it is the first (longest-chain) task
    of its bin. One task alone spreads over every bin (C = ceil(groups /
    n_bins)): its one table is all there is."""
    n = len(groups)
    if n == 1:
        return max(1, -(-groups[0] // n_bins)), [0], {0: 0}, {0: True}
    # sorting also reorders the mantissa groups, which follow the task array:
    # a layer of seven one-chain tensors decoded 1.4 % slower with its longest
    # tensors' buckets dispatched first than in the caller's order
    idx = list(range(n)) if n <= n_bins else sorted(range(n), key=lambda i: (-chain_len[i], -groups[i], i))
    C = max(max(groups, default=1), -(-sum(groups) // n_bins), 1)
    while True:
        used, bins = [0] * n_bins, [[] for _ in range(n_bins)]
        for i in idx:
            j = min(range(n_bins), key=lambda b: (used[b], b))
            if used[j] + groups[i] > C:
                break
            bins[j].append(i)
            used[j] += groups[i]
        else:
            break
        C += 1
    order, begin, first = [], {}, {}
    for j, b in enumerate(bins):
        at = j * C
        for k, i in enumerate(b):
            order.append(i)
            begin[i], first[i] = at, k == 0
            at += groups[i]
    return C, order, begin, first


class RefBatch:
    """The wave-serial decode of several parsed blobs (a layer's
    reference-format tensors) as one bs_refcodec_decode_serial_batch launch:
    all their chains run side by side, the SE chains (the longest) first.
    items: [(plan, blob_ptr, out_ptr)], every plan accepted by serial_ok.
    Device buffers stay alive with this object until the decode launched from
    it has completed.

    The SE groups are laid out by xcd_bins, so each XCD decodes the SE chains
    of one tensor or a few. The first tensor of each bin, when it has at most
    256 live SE symbols, keeps its chains' state in scalar registers and reads
    a 4-byte table through the scalar cache (a 16 KB table: one per XCD stays
    resident, where seven tensors' tables spread over every XCD missed, an 8B
    layer taking 43-45 against 39-41 ms with LDS tables); the other tensors of
    the bin, and every mantissa chain, read LDS tables (the scalar cache
    measured no faster for mantissa chains). SE_SCALAR: "auto" (that rule),
    True (every eligible tensor) or False; MANT_SCALAR: bool."""

    SE_SCALAR = "auto"
    MANT_SCALAR = False

    def __init__(self, items: list, device):
        import torch
        L = _native.lib()
        for plan, _, _ in items:
            if not serial_ok(plan):
                raise ValueError("RefBatch: a tensor the wave-serial path does not take")
        per = int(L.bs_refcodec_serial_chains_per_group())
        groups = [-(-len(p.se_streams) // per) for p, _, _ in items]
        lens = [max(n for _, _, _, n in p.se_streams) for p, _, _ in items]
        C, order, begin, first = xcd_bins(groups, lens)
        arrays = []
        tasks = np.zeros(len(items), REF_TASK_DTYPE)
        mant_g = tile = stream = work = 0
        for i, it in enumerate(order):       # task array in grid order: every *_begin ascends
            plan, blob_ptr, out_ptr = items[it]
            arrays += _plan_arrays(plan, blob_ptr)
            ns, nb = len(plan.se_streams), len(plan.buckets)
            nt = max(1, len(plan.mant_freqs))
            tiles = int(L.bs_refcodec_serial_tiles(plan.n, ns))
            flags = FLAG_MANT_SCALAR if self.MANT_SCALAR else 0
            if arrays[-4].nbytes > 8 * M_SE and (self.SE_SCALAR is True or (self.SE_SCALAR == "auto" and first[it])):
                flags |= FLAG_SE_SCALAR        # the SE table carries its 4-byte form
            tasks[i] = (0, 0, 0, 0, 0, out_ptr, plan.n, work, ns, nb, nt, begin[it], tile, stream, mant_g, flags)
            work += (int(L.bs_refcodec_serial_work_bytes(plan.n, ns)) + 255) & ~255
            mant_g += -(-nb // per)
            tile, stream = tile + ns * tiles, stream + ns
        se_g = XCD_BINS * C
        size, offs = _layout(arrays + [tasks.view(np.uint8)])
        self.dev = torch.empty(size, dtype=torch.uint8, device=device)
        base = self.dev.data_ptr()
        for i in range(len(items)):        # descriptor pointers into the device buffer
            o = offs[5 * i: 5 * i + 5]
            for f, off in zip(("streams", "se_table", "bstart", "buckets", "mant_tables"), o):
                tasks[f][i] = base + off
        buf, _ = _pack(arrays + [tasks.view(np.uint8)])
        self.dev.copy_(torch.from_numpy(buf))
        self.p_tasks = base + offs[-1]
        self.n_tasks = len(items)
        self.totals = (se_g, mant_g, tile, stream)
        self.work = torch.empty(max(work, 256), dtype=torch.uint8, device=device)

    def launch(self, status_ptr: int, stream_ptr: int) -> None:
        if not self.n_tasks:
            return
        rc = _native.lib().bs_refcodec_decode_serial_batch(self.p_tasks, self.n_tasks, *self.totals,
                                                            self.work.data_ptr(), self.work.numel(), status_ptr,
                                                            stream_ptr)
        _native.check(rc, "bs_refcodec_decode_serial_batch")


class RefLaunch:
    """Device-side tables and descriptors of one parsed blob (kept alive until
    the decode launched from them has completed). A tensor of
    SERIAL_MIN_ELEMENTS or more decodes with one wavefront per chain (a
    one-task bs_refcodec_decode_serial_batch, whose tables are built for one
    output address: pass `out_ptr` here to build them before the first
    launch); a smaller one with one lane per chain (bs_refcodec_decode)."""

    def __init__(self, plan: RefPlan, blob_ptr: int, device, out_ptr: int | None = None):
        import torch
        self.n_streams, self.n_buckets = len(plan.se_streams), len(plan.buckets)
        self.n_tables = max(1, len(plan.mant_freqs))
        self.n = plan.n
        self.plan, self.blob_ptr, self.device = plan, blob_ptr, device
        self._batch = None
        self.serial = serial_ok(plan)
        if self.serial:
            if out_ptr is not None:
                self._batch = (out_ptr, RefBatch([(plan, blob_ptr, out_ptr)], device))
            return
        buf, offs = _pack(_plan_arrays(plan, blob_ptr))
        self.dev = torch.from_numpy(buf).to(device)
        base = self.dev.data_ptr()
        self.p_streams, self.p_se_table, self.p_bstart, self.p_buckets, self.p_tables = (base + o for o in offs)
        self.perm = torch.empty(max(plan.n, 1), dtype=torch.int32, device=device)

    def launch(self, out_ptr: int, status_ptr: int, stream_ptr: int) -> None:
        L = _native.lib()
        if self.serial:
            # a one-task batch (its tables and flags built once per output)
            if self._batch is None or self._batch[0] != out_ptr:
                self._batch = (out_ptr, RefBatch([(self.plan, self.blob_ptr, out_ptr)], self.device))
            self._batch[1].launch(status_ptr, stream_ptr)
            return
        rc = L.bs_refcodec_decode(self.p_streams, self.n_streams, self.p_se_table, self.p_bstart,
                                  self.p_buckets, self.n_buckets, self.p_tables, self.n_tables,
                                  out_ptr, self.n, self.perm.data_ptr(), status_ptr, stream_ptr)
        _native.check(rc, "bs_refcodec_decode")


ENCODER_IDS = {"bf16_parallel_v1": 0, "bf16_se_tans": 1, "bf16_se_single_kernel": 2}   # BS_REF_*


def encode_host(codec: str, raw, n_streams: int = 128, threads: int | None = None) -> bytes:
    """The reference encoder's blob for bf16 bytes `raw`, written by the host
    encoder of this library (bs_refcodec_encode). Odd byte counts raise
    ValueError, as the reference's encoders do."""
    import ctypes
    import os
    mv = memoryview(raw).cast("B")
    if len(mv) % 2:
        raise ValueError(f"BF16 byte length must be even, got {len(mv)}")
    words = np.frombuffer(mv, dtype=np.uint16)
    n = int(words.size)
    if n == 0:
        return b""
    L = _native.lib()
    cid = ENCODER_IDS[codec]
    # bf16_parallel.py:195 clamps N = max(1, min(n_streams, n)); the C encoder
    # clamps the upper side, a count below 1 is clamped here (it takes a u32)
    n_streams = min(max(1, int(n_streams)), n)
    cap = int(L.bs_refcodec_encode_bound(cid, n, n_streams))
    out = np.empty(cap, np.uint8)
    olen = ctypes.c_uint64(0)
    src = np.ascontiguousarray(words)
    rc = L.bs_refcodec_encode(cid, src.ctypes.data, n, n_streams, out.ctypes.data, cap, ctypes.byref(olen),
                              threads or min(16, os.cpu_count() or 1))
    if rc == _native.BS_ERR_FORMAT:
        raise ValueError(f"{codec}: frequency quantisation failed")
    _native.check(rc, "bs_refcodec_encode")
    return out[:olen.value].tobytes()


def decode_host(codec: str, blob: bytes, n_weights: int) -> bytes:
    """Reference-shaped decode: host bytes in, host bytes out; decoded on the GPU."""
    import torch
    from ..device import StatusWord, require_gpu, stream_ptr, upload_bytes
    if n_weights == 0 or len(blob) == 0:
        return b""
    plan = PARSERS[codec](bytes(blob), n_weights)
    dev = require_gpu()
    d_blob = upload_bytes(blob, dev)
    out = torch.empty(n_weights, dtype=torch.int16, device=dev)
    st = StatusWord(dev)
    launch = RefLaunch(plan, d_blob.data_ptr(), dev, out.data_ptr())
    launch.launch(out.data_ptr(), st.ptr, stream_ptr(None, dev))
    torch.cuda.synchronize(dev)
    st.check(codec)
    return out.cpu().numpy().tobytes()


__all__ = ["PARSERS", "RefBatch", "RefLaunch", "RefPlan", "serial_ok", "decode_host", "encode_host", "parse_parallel", "parse_tans",
           "parse_single_kernel", "decode_table_se", "decode_table_se_scalar", "decode_table_mant"]
