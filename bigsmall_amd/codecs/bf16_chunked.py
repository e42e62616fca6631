"""`bf16_chunked_v1` / `fp8_chunked_v1` (rANS) and `bf16_chunked_tans_v1` /
`fp8_chunked_tans_v1` (tANS): the engine's GPU-native codecs.

A tensor is cut into chunks of `lanes` x `steps` elements (128 x 432 by
default). Each chunk is `lanes` interleaved entropy-coder states (lanes / 64
per wavefront lane) over the tensor's exponent (or exact-value) symbols,
sharing one stream per chunk, plus raw sign|mantissa bytes. The rANS codecs
share a 16-bit renormalisation word stream; the tANS codecs a bit stream
that each state reads its table-given bit count from. fp8 tensors code
pairs of exponent fields as one symbol when that is smaller (plane mode 3).
Full chunks own 512-element units of the tensor interleaved across all of
them (chunk c: units c, nf + c, 2 nf + c, ...), so the chunks a launch
decodes side by side write neighbouring addresses; their dense planes are
interleaved the same way in one region of the blob. The blob layout is
documented in bigsmall_amd/csrc/bsck_decode.hip.

Plugin shape of the reference codec API (bigsmall/codec_registry.py:39-42):
    encode(raw: bytes, **ctx) -> (blob, extras)
    decode(blob: bytes, extras: dict, n_weights: int) -> bytes
plus the device entry points the engine itself uses (`decode_into`).
Decoding runs only on the GPU.
"""
from __future__ import annotations

import contextlib
import ctypes
import os

import numpy as np

from .. import _native
from ..device import (ChunkBatch, ChunkJob, StatusWord, inspect_chunk_header, require_gpu, stream_ptr,
                      upload_bytes, upload_bytes_async)

CODEC_BF16 = "bf16_chunked_v1"
CODEC_FP8 = "fp8_chunked_v1"
CODEC_BF16_TANS = "bf16_chunked_tans_v1"
CODEC_FP8_TANS = "fp8_chunked_tans_v1"
CODER_RANS, CODER_TANS = 0, 2
# tANS chunks whose initial states are a u32 array before the stream (coder 2
# keeps them as 12-bit fields at the stream head): the layout of earlier
# blobs, still decoded, and written only on request
CODER_TANS_STATE_ARRAY = 1
# 432 steps x 128 states = 55,296 elements per chunk: a Llama-3-8B-shaped
# layer is 3,948 chunks in 497 eight-wave workgroups, one dispatch round of
# the 512 workgroup slots of 256 CUs (two per CU), with 15 CUs holding one
# workgroup (32 at 448 steps; 416 steps need 516 workgroups, four of them in
# a second round). Measured
# on MI355X with the decoder's progress priority: 151.1 us per layer against
# 154.9 us at 448 steps; the ratio cost is +0.013 pp (one 32-bit initial
# state per 432 elements).
DEFAULT_STEPS = 432
DEFAULT_LANES = 128
# tANS chunks: four states per wavefront lane over half the steps (the same
# elements per chunk, rounded up to 16 steps). The step's dependency chain
# (table read, wavefront prefix sum, window read) then overlaps across four
# states: on MI355X the half-zeros 8192^2 tensor (64-step chunks) decodes
# 5 % faster than at 128 lanes x 128 steps and the pruned 8B layer (224
# steps) 2.6 % faster than at 128 x 432, and with 12-bit head states the
# blob is still smaller than at 128 lanes with u32 states.
TANS_LANES = 256


def tans_steps(steps: int) -> int:
    """Steps per tANS chunk for a rANS chunk of `steps` steps at 128 lanes."""
    return max(16, -(-steps // 32) * 16)
MODE_AUTO, MODE_EXACT, MODE_DENSE, MODE_COMPACT, MODE_PAIRS = -1, 0, 1, 2, 3


def _threads() -> int:
    return max(1, min(os.cpu_count() or 1, 16))


def encode_array(arr: np.ndarray, steps: int = DEFAULT_STEPS, mode: int = MODE_AUTO,
                 threads: int | None = None, lanes: int = DEFAULT_LANES, coder: int = CODER_RANS) -> bytes:
    """Encode a uint16 (bf16 words) or uint8 (fp8 bytes) array with the rANS
    coder (CODER_RANS) or the tANS coder (CODER_TANS; CODER_TANS_STATE_ARRAY
    writes the earlier layout of its initial states)."""
    a = np.ascontiguousarray(arr)
    if a.dtype not in (np.uint16, np.uint8):
        raise TypeError("encode_array expects uint16 (bf16 bit patterns) or uint8 (fp8 bytes)")
    eb = a.dtype.itemsize
    n = a.size
    if n == 0:
        return b""
    L = _native.lib()
    bound = ctypes.c_uint64()
    _native.check(L.bs_chunk_encode_bound_ex(n, eb, lanes, steps, coder, ctypes.byref(bound)),
                  "bs_chunk_encode_bound_ex")
    out = np.empty(bound.value, np.uint8)
    olen = ctypes.c_uint64()
    _native.check(L.bs_chunk_encode_ex(a.ctypes.data, n, eb, lanes, steps, mode, coder, out.ctypes.data, bound.value,
                                       ctypes.byref(olen), threads or _threads()), "bs_chunk_encode_ex")
    return out[: olen.value].tobytes()


# bs_encode_task (include/bigsmall_hip.h): 56 bytes; seg_len 0 = contiguous words
ENCODE_TASK_DTYPE = np.dtype([("src", "<u8"), ("n", "<u8"), ("dst", "<u8"), ("cap", "<u8"),
                              ("chunk_begin", "<u4"), ("n_chunks", "<u4"), ("seg_len", "<u8"), ("seg_stride", "<u8")])
assert ENCODE_TASK_DTYPE.itemsize == 56
GPU_ENCODE_LANES = 128


SPAN_DTYPE = np.dtype([("src", "<u8"), ("dst", "<u8"), ("len", "<u8")])     # bs_span


def _encode_bound(n: int, steps: int, cache: dict) -> int:
    if n not in cache:
        bound = ctypes.c_uint64()
        _native.check(_native.lib().bs_chunk_encode_bound(max(n, 1), 2, GPU_ENCODE_LANES, steps, ctypes.byref(bound)),
                      "bs_chunk_encode_bound")
        cache[n] = int(bound.value)
    return cache[n]


def _run_encode(dev, tasks: np.ndarray, total_chunks: int, steps: int, stream):
    """bs_chunk_encode_gpu over `tasks` (ENCODE_TASK_DTYPE, sorted by
    chunk_begin); waits for it and returns (blob lengths as int64 numpy, the
    checked status word)."""
    import torch
    L = _native.lib()
    # one upload: a zeroed result area (the status word, the low half of
    # element 0, then the lengths) and the task table after it; one copy on
    # the encode's stream brings the results back
    nres = 8 * (1 + len(tasks))
    toff = (nres + 255) & ~255                          # the task table stays 256-byte aligned
    buf = np.zeros(toff + tasks.nbytes, np.uint8)
    buf[toff:] = tasks.view(np.uint8)
    d_buf = upload_bytes_async(buf, dev, stream)
    res = d_buf[:nres].view(torch.int64)
    d_tasks = d_buf[toff:]
    wb = int(L.bs_chunk_encode_gpu_work_bytes(len(tasks), total_chunks, steps))
    with torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext():
        work = torch.empty(max(wb, 256), dtype=torch.uint8, device=dev)
    st = StatusWord(view=res[:1].view(torch.int32)[:1])
    _native.check(L.bs_chunk_encode_gpu(d_tasks.data_ptr(), len(tasks), total_chunks, steps, work.data_ptr(), wb,
                                        res[1:].data_ptr(), st.ptr, stream_ptr(stream, dev)), "bs_chunk_encode_gpu")
    with torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext():
        host = res.cpu().numpy()
    if int(host[0]) & 0xFFFFFFFF:
        st.check("bf16_chunked GPU encode")
    return host[1:], st


def _pack(arena, src_offs: np.ndarray, lens: np.ndarray, dev, st: StatusWord, stream):
    """Copy the blobs arena[src_offs[i]:+lens[i]] back to back into a new
    tensor with one bs_copy_spans launch; returns (tight, offsets)."""
    import torch
    if np.any(lens % 16):
        raise RuntimeError("GPU encoder returned a blob length that is not a multiple of 16")
    offs = np.zeros(len(lens), np.int64)
    np.cumsum(lens[:-1], out=offs[1:])
    total = int(lens.sum())
    with torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext():
        tight = torch.empty(max(total, 256), dtype=torch.uint8, device=dev)     # owned by the copy's stream
    live = lens > 0
    if live.any():
        spans = np.zeros(int(live.sum()), SPAN_DTYPE)
        spans["src"] = arena.data_ptr() + src_offs[live].astype(np.uint64)
        spans["dst"] = tight.data_ptr() + offs[live].astype(np.uint64)
        spans["len"] = lens[live]
        d_spans = upload_bytes_async(spans.view(np.uint8), dev, stream)
        _native.check(_native.lib().bs_copy_spans(d_spans.data_ptr(), len(spans), int(lens.max()), st.ptr,
                                                  stream_ptr(stream, dev)), "bs_copy_spans")
        if stream is not None:        # the launch's inputs stay allocated until it has run
            for t in (d_spans, arena, st.t):
                t.record_stream(stream)
    return tight, offs


def encode_device(tensors, steps: int = DEFAULT_STEPS, stream=None, compact: bool = True):
    """Encode device-resident bf16 tensors on the GPU (dense plane mode, 128
    states per chunk); the blobs equal encode_array(words, steps, MODE_DENSE).

    Returns (arena, [(offset, length), ...]): every blob lives in one device
    uint8 tensor. With compact=True the blobs are packed back to back (every
    blob length is a multiple of 16, so each stays 16-byte aligned); with
    compact=False each keeps its worst-case slot at a 256-byte aligned offset
    (no copy after encoding)."""
    import torch
    if not tensors:
        return None, []
    dev = require_gpu(tensors[0].device)
    per = GPU_ENCODE_LANES * steps
    srcs, slots, cap_total = [], [], 0
    bounds: dict[int, int] = {}
    for t in tensors:
        if t.dtype != torch.bfloat16 or t.device != dev:
            raise ValueError("encode_device expects bf16 tensors on one GPU")
        t = t.contiguous()
        if t.data_ptr() % 4:
            t = t.clone()
        bound = _encode_bound(t.numel(), steps, bounds)
        srcs.append(t)
        slots.append((cap_total, bound))
        cap_total += (bound + 255) & ~255
    arena = torch.empty(max(cap_total, 256), dtype=torch.uint8, device=dev)
    live = [i for i, t in enumerate(srcs) if t.numel() > 0]
    tasks = np.zeros(len(live), ENCODE_TASK_DTYPE)
    chunk = 0
    for k, i in enumerate(live):
        n = srcs[i].numel()
        nch = (n + per - 1) // per
        tasks[k] = (srcs[i].data_ptr(), n, arena.data_ptr() + slots[i][0], slots[i][1], chunk, nch, 0, 0)
        chunk += nch
    lens = np.zeros(len(srcs), np.int64)
    st = None
    if live:
        got, st = _run_encode(dev, tasks, chunk, steps, stream)
        lens[live] = got
    if not compact:
        return arena, [(slots[i][0], int(lens[i])) for i in range(len(srcs))]
    if st is None:
        return torch.empty(256, dtype=torch.uint8, device=dev), [(0, 0)] * len(srcs)
    tight, offs = _pack(arena, np.array([s[0] for s in slots], np.int64), lens, dev, st, stream)
    return tight, list(zip(offs.tolist(), lens.tolist()))


def encode_device_rows(groups, steps: int = DEFAULT_STEPS, stream=None):
    """encode_device for many equal-size pieces: every row of each bf16
    device tensor in `groups` becomes one blob (e.g. the 256-token blocks of a
    KV layer), with the task table built without a per-row Python loop. A
    group is a contiguous 2-D tensor [rows, n], or a 3-D view [rows, segments,
    seg_len] whose segments are contiguous (a block of tokens of a [heads,
    tokens, dim] tensor: rows = blocks, segments = heads), read in place:
    seg_len a multiple of 512, segment starts a multiple of 8 words apart.
    Returns (arena, offsets, lengths): blobs packed back to back in one device
    uint8 tensor, offsets and lengths as int64 numpy arrays in row order over
    all groups."""
    import torch
    if not groups:
        return None, np.zeros(0, np.int64), np.zeros(0, np.int64)
    dev = require_gpu(groups[0].device)
    per = GPU_ENCODE_LANES * steps
    bounds: dict[int, int] = {}
    shapes, cap_total = [], 0
    for g in groups:
        if g.dtype != torch.bfloat16 or g.device != dev or g.dim() not in (2, 3):
            raise ValueError("encode_device_rows expects 2-D or 3-D bf16 tensors on one GPU")
        if g.dim() == 2:
            if not g.is_contiguous():
                raise ValueError("encode_device_rows expects 2-D groups to be contiguous")
            rows, n = g.shape
            row_stride, seg = n, (0, 0)
        else:
            rows, nseg, seg_len = g.shape
            n = nseg * seg_len
            if rows and n and (g.stride(2) != 1 or seg_len % 512 or
                               (nseg > 1 and (g.stride(1) % 8 or g.stride(1) < seg_len or
                                              (nseg - 1) * g.stride(1) + seg_len > 2 ** 32))):
                raise ValueError("encode_device_rows: a 3-D group needs contiguous segments of a multiple of "
                                 "512 words whose starts are a multiple of 8 words apart")
            row_stride, seg = g.stride(0), ((seg_len, g.stride(1)) if nseg > 1 else (0, 0))
        if rows and n and (g.data_ptr() % 4 or (rows > 1 and row_stride % 2)):
            raise ValueError("encode_device_rows needs 4-byte aligned rows (an even row length)")
        slot = (_encode_bound(n, steps, bounds) + 255) & ~255 if rows and n else 0
        shapes.append((rows, n, slot, cap_total, row_stride, seg))
        cap_total += rows * slot
    arena = torch.empty(max(cap_total, 256), dtype=torch.uint8, device=dev)
    n_rows = sum(r for r, *_ in shapes)
    lens = np.zeros(n_rows, np.int64)
    src_offs = np.zeros(n_rows, np.int64)
    parts, chunk, r0 = [], 0, 0
    for g, (rows, n, slot, base, row_stride, seg) in zip(groups, shapes):
        idx = np.arange(rows, dtype=np.uint64)
        src_offs[r0:r0 + rows] = base + idx.astype(np.int64) * slot
        if rows and n:
            nch = (n + per - 1) // per
            t = np.zeros(rows, ENCODE_TASK_DTYPE)
            t["src"] = g.data_ptr() + idx * np.uint64(2 * row_stride)
            t["seg_len"], t["seg_stride"] = seg
            t["n"] = n
            t["dst"] = arena.data_ptr() + np.uint64(base) + idx * np.uint64(slot)
            t["cap"] = _encode_bound(n, steps, bounds)
            t["chunk_begin"] = chunk + idx.astype(np.uint32) * np.uint32(nch)
            t["n_chunks"] = nch
            parts.append((r0, t))
            chunk += rows * nch
        r0 += rows
    if not parts:
        return torch.empty(256, dtype=torch.uint8, device=dev), np.zeros(n_rows, np.int64), lens
    tasks = np.concatenate([t for _, t in parts])
    if chunk >= 2 ** 32:
        raise ValueError("encode_device_rows: more than 2^32 chunks in one batch")
    got, st = _run_encode(dev, tasks, chunk, steps, stream)
    k = 0
    for r, t in parts:
        lens[r:r + len(t)] = got[k:k + len(t)]
        k += len(t)
    tight, offs = _pack(arena, src_offs, lens, dev, st, stream)
    return tight, offs, lens


def encode(raw: bytes, steps: int = DEFAULT_STEPS, mode: int = MODE_AUTO, **_) -> tuple[bytes, dict]:
    """bf16 raw bytes -> (blob, extras)."""
    if len(raw) % 2:
        raise ValueError(f"BF16 byte length must be even, got {len(raw)}")
    blob = encode_array(np.frombuffer(raw, dtype="<u2"), steps=steps, mode=mode)
    return blob, {"steps": steps}


def encode_fp8(raw: bytes, steps: int = DEFAULT_STEPS, mode: int = MODE_AUTO, **_) -> tuple[bytes, dict]:
    """fp8 raw bytes -> (blob, extras): byte symbols or exponent-pair symbols,
    whichever codes smaller."""
    blob = encode_array(np.frombuffer(raw, dtype=np.uint8), steps=steps, mode=mode)
    return blob, {"steps": steps}


def encode_tans(raw: bytes, steps: int = DEFAULT_STEPS, mode: int = MODE_AUTO, **_) -> tuple[bytes, dict]:
    """bf16 raw bytes -> (blob, extras), tANS coder (TANS_LANES states per
    chunk over tans_steps(steps) steps)."""
    if len(raw) % 2:
        raise ValueError(f"BF16 byte length must be even, got {len(raw)}")
    ts = tans_steps(steps)
    blob = encode_array(np.frombuffer(raw, dtype="<u2"), steps=ts, mode=mode, lanes=TANS_LANES, coder=CODER_TANS)
    return blob, {"steps": ts}


def encode_fp8_tans(raw: bytes, steps: int = DEFAULT_STEPS, mode: int = MODE_AUTO, **_) -> tuple[bytes, dict]:
    """fp8 raw bytes -> (blob, extras), tANS coder (geometry as encode_tans)."""
    ts = tans_steps(steps)
    blob = encode_array(np.frombuffer(raw, dtype=np.uint8), steps=ts, mode=mode, lanes=TANS_LANES, coder=CODER_TANS)
    return blob, {"steps": ts}


def info(blob: bytes) -> _native.BsChunkInfo:
    return inspect_chunk_header(bytes(blob[:32]))


def decode_into(d_blob, blob_bytes: int, out, n: int, status: StatusWord | None = None, stream=None) -> StatusWord:
    """Decode a device-resident blob (uint8 tensor or address) into `out`
    (a device tensor of n elements of the blob's element size). Asynchronous
    on `stream`; returns the status word to check after synchronising."""
    import torch
    if n == 0:
        return status or StatusWord(out.device)
    ptr = d_blob.data_ptr() if isinstance(d_blob, torch.Tensor) else int(d_blob)
    head = (d_blob[:32].cpu().numpy().tobytes() if isinstance(d_blob, torch.Tensor) else None)
    if head is None:
        raise ValueError("decode_into needs the blob tensor (its header sizes the launch)")
    inf = inspect_chunk_header(head)
    if inf.n != n:
        raise ValueError(f"bf16_chunked: weight count mismatch ({inf.n} vs {n})")
    if out.numel() * out.element_size() < n * inf.elem_bytes:
        raise ValueError("output tensor too small")
    st = status or StatusWord(out.device)
    batch = ChunkBatch([ChunkJob(ptr, blob_bytes, out.data_ptr(), n, inf.n_chunks, inf.plane_mode)], out.device)
    batch.launch(st, stream)
    return st


def decode(blob: bytes, extras: dict, n_weights: int, elem_bytes: int = 2) -> bytes:
    """Reference-shaped plugin decode: host bytes in, host bytes out; the
    decode itself runs on the GPU."""
    import torch
    if n_weights == 0 or len(blob) == 0:
        return b""
    dev = require_gpu()
    inf = info(blob)
    if inf.n != n_weights:
        raise ValueError(f"bf16_chunked: weight count mismatch ({inf.n} vs {n_weights})")
    d_blob = upload_bytes(blob, dev)
    out = torch.empty(n_weights * inf.elem_bytes, dtype=torch.uint8, device=dev)
    st = decode_into(d_blob, len(blob), out, n_weights)
    torch.cuda.synchronize(dev)
    st.check(CODEC_BF16 if inf.elem_bytes == 2 else CODEC_FP8)
    return out.cpu().numpy().tobytes()


def decode_fp8(blob: bytes, extras: dict, n_weights: int) -> bytes:
    return decode(blob, extras, n_weights, elem_bytes=1)
