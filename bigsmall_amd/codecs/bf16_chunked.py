"""`bf16_chunked_v1` / `fp8_chunked_v1`: the engine's GPU-native codec.

A tensor is cut into chunks of 64 x `steps` elements. Each chunk is 64
interleaved rANS streams (one per wavefront lane) over the tensor's exponent
(or exact-value) symbols, sharing one 16-bit renormalisation word stream, plus
a plane of raw sign|mantissa bytes. The blob layout is documented in
bigsmall_amd/csrc/bsck_decode.hip.

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
                      upload_bytes)

CODEC_BF16 = "bf16_chunked_v1"
CODEC_FP8 = "fp8_chunked_v1"
# 448 steps x 128 states = 57,344 elements per chunk: a 14336x4096 matrix is
# 1024 chunks (128 full 8-wave workgroups) and a Llama-3-8B-shaped layer fits
# in one round of 480 workgroups on 256 CUs (two per CU). Measured on MI355X:
# 0.175 ms/layer vs 0.184 at 512 steps; the ratio cost of the shorter chunks
# is +0.05 pp (one 32-bit initial state per 448 elements).
DEFAULT_STEPS = 448
DEFAULT_LANES = 128
MODE_AUTO, MODE_EXACT, MODE_DENSE, MODE_COMPACT = -1, 0, 1, 2


def _threads() -> int:
    return max(1, min(os.cpu_count() or 1, 16))


def encode_array(arr: np.ndarray, steps: int = DEFAULT_STEPS, mode: int = MODE_AUTO,
                 threads: int | None = None, lanes: int = DEFAULT_LANES) -> bytes:
    """Encode a uint16 (bf16 words) or uint8 (fp8 bytes) array."""
    a = np.ascontiguousarray(arr)
    if a.dtype not in (np.uint16, np.uint8):
        raise TypeError("encode_array expects uint16 (bf16 bit patterns) or uint8 (fp8 bytes)")
    eb = a.dtype.itemsize
    n = a.size
    if n == 0:
        return b""
    L = _native.lib()
    bound = ctypes.c_uint64()
    _native.check(L.bs_chunk_encode_bound(n, eb, lanes, steps, ctypes.byref(bound)), "bs_chunk_encode_bound")
    out = np.empty(bound.value, np.uint8)
    olen = ctypes.c_uint64()
    _native.check(L.bs_chunk_encode(a.ctypes.data, n, eb, lanes, steps, mode, out.ctypes.data, bound.value,
                                    ctypes.byref(olen), threads or _threads()), "bs_chunk_encode")
    return out[: olen.value].tobytes()


# bs_encode_task (include/bigsmall_hip.h): 40 bytes
ENCODE_TASK_DTYPE = np.dtype([("src", "<u8"), ("n", "<u8"), ("dst", "<u8"), ("cap", "<u8"),
                              ("chunk_begin", "<u4"), ("n_chunks", "<u4")])
assert ENCODE_TASK_DTYPE.itemsize == 40
GPU_ENCODE_LANES = 128


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
    L = _native.lib()
    per = GPU_ENCODE_LANES * steps
    srcs, slots, cap_total = [], [], 0
    bounds: dict[int, int] = {}
    for t in tensors:
        if t.dtype != torch.bfloat16 or t.device != dev:
            raise ValueError("encode_device expects bf16 tensors on one GPU")
        t = t.contiguous()
        if t.data_ptr() % 4:
            t = t.clone()
        n = t.numel()
        if n not in bounds:
            bound = ctypes.c_uint64()
            _native.check(L.bs_chunk_encode_bound(max(n, 1), 2, GPU_ENCODE_LANES, steps, ctypes.byref(bound)),
                          "bs_chunk_encode_bound")
            bounds[n] = int(bound.value)
        srcs.append(t)
        slots.append((cap_total, bounds[n]))
        cap_total += (bounds[n] + 255) & ~255
    arena = torch.empty(max(cap_total, 256), dtype=torch.uint8, device=dev)
    live = [i for i, t in enumerate(srcs) if t.numel() > 0]
    tasks = np.zeros(len(live), ENCODE_TASK_DTYPE)
    chunk = 0
    for k, i in enumerate(live):
        n = srcs[i].numel()
        nch = (n + per - 1) // per
        tasks[k] = (srcs[i].data_ptr(), n, arena.data_ptr() + slots[i][0], slots[i][1], chunk, nch)
        chunk += nch
    lens = [0] * len(srcs)
    if live:
        d_tasks = upload_bytes(tasks.view(np.uint8), dev)
        wb = int(L.bs_chunk_encode_gpu_work_bytes(len(live), chunk, steps))
        work = torch.empty(max(wb, 256), dtype=torch.uint8, device=dev)
        out_len = torch.zeros(len(live), dtype=torch.int64, device=dev)
        st = StatusWord(dev)
        _native.check(L.bs_chunk_encode_gpu(d_tasks.data_ptr(), len(live), chunk, steps, work.data_ptr(), wb,
                                            out_len.data_ptr(), st.ptr, stream_ptr(stream, dev)),
                      "bs_chunk_encode_gpu")
        torch.cuda.synchronize(dev)
        st.check("bf16_chunked GPU encode")
        host_lens = out_len.cpu().tolist()
        for k, i in enumerate(live):
            lens[i] = int(host_lens[k])
    if not compact:
        return arena, [(slots[i][0], lens[i]) for i in range(len(srcs))]
    offs, pos = [], 0
    for ln in lens:
        if ln % 16:
            raise RuntimeError(f"GPU encoder returned a blob length {ln} that is not a multiple of 16")
        offs.append(pos)
        pos += ln
    # slots start at multiples of 256 and lengths are multiples of 16: copy as
    # 8-byte words, in one batched kernel rather than one copy per blob
    words = arena.view(torch.int64)
    parts = [words[slots[i][0] // 8:(slots[i][0] + ln) // 8] for i, ln in enumerate(lens) if ln]
    if not parts:
        return torch.empty(256, dtype=torch.uint8, device=dev), list(zip(offs, lens))
    with torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext():
        tight = torch.cat(parts).view(torch.uint8)
    return tight, list(zip(offs, lens))


def encode(raw: bytes, steps: int = DEFAULT_STEPS, mode: int = MODE_AUTO, **_) -> tuple[bytes, dict]:
    """bf16 raw bytes -> (blob, extras)."""
    if len(raw) % 2:
        raise ValueError(f"BF16 byte length must be even, got {len(raw)}")
    blob = encode_array(np.frombuffer(raw, dtype="<u2"), steps=steps, mode=mode)
    return blob, {"steps": steps}


def encode_fp8(raw: bytes, steps: int = DEFAULT_STEPS, **_) -> tuple[bytes, dict]:
    blob = encode_array(np.frombuffer(raw, dtype=np.uint8), steps=steps, mode=MODE_EXACT)
    return blob, {"steps": steps}


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
