"""Device plumbing for the decode engine: streams, uploads, status words and
batched BSCK launches. torch provides device memory and streams; all decoding
happens in the HIP kernels of libbigsmall_hip.so.
"""
from __future__ import annotations

import contextlib

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _native
from .exceptions import DecodeError

# bs_chunk_task (include/bigsmall_hip.h): 40 bytes, 8-byte aligned
TASK_DTYPE = np.dtype([("blob", "<u8"), ("blob_bytes", "<u8"), ("out", "<u8"), ("n", "<u8"),
                       ("wg_begin", "<u4"), ("n_chunks", "<u4")])
assert TASK_DTYPE.itemsize == 40


def require_gpu(device=None):
    """Return a torch.device for decoding; raise if no ROCm GPU is present."""
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("bigsmall_amd decodes on an AMD GPU (MI355X); no ROCm device is available")
    dev = torch.device(device if device is not None else "cuda")
    if dev.type != "cuda":
        raise ValueError(f"decode device must be a ROCm GPU, got {dev}")
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


def stream_ptr(stream=None, device=None) -> int:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream(device)
    return int(s.cuda_stream)


def upload_bytes(data, device, align: int = 256):
    """Copy host bytes to a fresh device uint8 tensor (allocator blocks are
    >= 256-byte aligned)."""
    import torch
    arr = np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray) else data.view(np.uint8).reshape(-1)
    host = torch.from_numpy(arr.copy() if not arr.flags.writeable else arr)
    out = torch.empty(len(arr), dtype=torch.uint8, device=device)
    if len(arr):
        out.copy_(host)
    assert out.data_ptr() % align == 0
    return out


def upload_bytes_async(data, device, stream=None):
    """upload_bytes through pinned staging with a non-blocking copy on
    `stream` (the current stream if None): the host does not wait for the
    copy, or for the work queued before it; later work on that stream sees the
    bytes. The staging block comes from torch's pinned caching allocator,
    which keeps it from reuse until the copy has run."""
    import torch
    arr = np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray) else data.view(np.uint8).reshape(-1)
    out = torch.empty(len(arr), dtype=torch.uint8, device=device)
    if len(arr):
        host = torch.empty(len(arr), dtype=torch.uint8, pin_memory=True)
        host.numpy()[:] = arr
        with torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext():
            out.copy_(host, non_blocking=True)
        if stream is not None:
            out.record_stream(stream)
    return out


class StatusWord:
    """Device int32 that kernels OR their BS_DEV_* bits into."""

    def __init__(self, device=None, view=None):
        """A new zeroed word on `device`, or `view`: an int32 element of
        another device buffer that is already zero."""
        import torch
        self.t = view if view is not None else torch.zeros(1, dtype=torch.int32, device=device)

    @property
    def ptr(self) -> int:
        return self.t.data_ptr()

    def reset(self):
        self.t.zero_()

    def check(self, what: str = "decode") -> None:
        v = int(self.t.item())
        if v:
            names = [n for b, n in [(_native.BS_DEV_ERR_HEADER, "bad header"), (_native.BS_DEV_ERR_COUNT, "count mismatch"),
                                    (_native.BS_DEV_ERR_BOUNDS, "section out of bounds"),
                                    (_native.BS_DEV_ERR_STREAM, "corrupt entropy-coded stream")] if v & b]
            raise DecodeError(f"{what}: device integrity check failed ({', '.join(names)}; status=0x{v:x})")


@dataclass
class ChunkJob:
    """One BSCK blob to decode: device blob address/length, output address, counts."""
    blob_ptr: int
    blob_bytes: int
    out_ptr: int
    n: int
    n_chunks: int
    plane_mode: int = 2


def inspect_chunk_header(blob_head: bytes):
    """Parse a BSCK header. A malformed or truncated header is a data error:
    ValueError, as the reference raises for bad magic or counts
    (bigsmall/codecs/bf16_parallel.py:153-163)."""
    info = _native.BsChunkInfo()
    if len(blob_head) < 32:
        raise ValueError(f"bf16_chunked: blob too short for its header ({len(blob_head)} bytes)")
    buf = (ctypes.c_uint8 * len(blob_head)).from_buffer_copy(blob_head)
    rc = _native.lib().bs_chunk_inspect(ctypes.addressof(buf), len(blob_head), ctypes.byref(info))
    if rc == _native.BS_ERR_FORMAT:
        raise ValueError("bf16_chunked: malformed blob header")
    _native.check(rc, "bs_chunk_inspect")
    return info


class ChunkBatch:
    """A prepared batched launch: a device array of bs_chunk_task and its grid
    size. Reusable: launch() may be called repeatedly (e.g. for timing)."""

    def __init__(self, jobs: list[ChunkJob], device):
        import torch
        L = _native.lib()
        per = L.bs_chunk_chunks_per_group()
        tasks = np.zeros(len(jobs), TASK_DTYPE)
        wg = 0
        for i, j in enumerate(jobs):
            if j.blob_ptr % 16 or j.out_ptr % 16:
                raise ValueError("BSCK blobs and their outputs must be 16-byte aligned on the device")
            tasks[i] = (j.blob_ptr, j.blob_bytes, j.out_ptr, j.n, wg, j.n_chunks)
            wg += (j.n_chunks + per - 1) // per
        self.n_tasks = len(jobs)
        self.max_mode = max((j.plane_mode for j in jobs), default=0)
        self.total_groups = wg
        self.jobs = jobs
        self.tasks_dev = torch.from_numpy(tasks.view(np.uint8).copy()).to(device)

    def launch(self, status: StatusWord, stream=None) -> None:
        if self.n_tasks == 0:
            return
        rc = _native.lib().bs_chunk_decode_batch(self.tasks_dev.data_ptr(), self.n_tasks, self.total_groups,
                                                 self.max_mode, status.ptr, stream_ptr(stream))
        _native.check(rc, "bs_chunk_decode_batch")
