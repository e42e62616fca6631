"""Zstandard-coded container entries, decoded on the GPU (csrc/zstd_decode.hip).

The reference writes these with the `zstandard` package and decodes them on
the host:
  - "zstd": the tensor's bytes as one zstd frame (bigsmall/codecs/generic.py:9-18;
    dispatched at bigsmall/decoder.py:80-81);
  - "special" with special_kind "lowcard": the distinct element values and a
    zstd frame of one uint8 index per element (bigsmall/codecs/special.py:23-85);
  - "zstd_xor_delta": a zstd frame of the XOR difference to a base model's
    tensor (bigsmall/decoder.py:88-90; applied by decompress_delta, :190-198).
Here the host only reads the lowcard framing; the frames are decoded by
bs_zstd_decode and the lowcard indices expanded by bs_lut_expand.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

from .. import _native
from ..device import StatusWord, require_gpu, stream_ptr, upload_bytes

ZSTD_TASK_DTYPE = np.dtype([("src", "<u8"), ("src_len", "<u8"), ("dst", "<u8"), ("dst_len", "<u8"),
                            ("xor_src", "<u8")])
LUT_TASK_DTYPE = np.dtype([("idx", "<u8"), ("lut", "<u8"), ("out", "<u8"), ("n", "<u8"), ("n_lut", "<u4"),
                           ("item_bytes", "<u4")])
ZSTD_MAGIC = 0xFD2FB528


@dataclass
class Lowcard:
    """Byte layout of a lowcard blob (bigsmall/codecs/special.py:58-64):
    [u8 item_bytes][u8 n_unique][n_unique x item_bytes values][u32 idx_len]
    [idx_len bytes: zstd frame of uint8 indices][u32 n_elem]."""
    item_bytes: int
    n_unique: int
    lut_off: int
    idx_off: int
    idx_len: int
    n_elem: int


def parse_lowcard(blob) -> Lowcard:
    b = memoryview(blob).cast("B")
    if len(b) < 2:
        raise ValueError("lowcard blob shorter than its 2-byte header")
    ib, nu = b[0], b[1]
    p = 2 + nu * ib
    if len(b) < p + 4:
        raise ValueError("lowcard blob truncated in its value table")
    idx_len, = struct.unpack_from("<I", b, p)
    idx_off = p + 4
    if len(b) < idx_off + idx_len + 4:
        raise ValueError("lowcard blob truncated in its index stream")
    n_elem, = struct.unpack_from("<I", b, idx_off + idx_len)
    return Lowcard(ib, nu, 2, idx_off, idx_len, n_elem)


def frame_content_size(blob) -> int | None:
    """Frame_Content_Size of the first zstd frame (RFC 8878 3.1.1.1.4), or
    None when the frame does not record it."""
    b = memoryview(blob).cast("B")
    if len(b) < 5 or struct.unpack_from("<I", b, 0)[0] != ZSTD_MAGIC:
        raise ValueError("not a zstd frame")
    fhd = b[4]
    fcs_flag, single, did = fhd >> 6, (fhd >> 5) & 1, fhd & 3
    fcs_bytes = (single if fcs_flag == 0 else {1: 2, 2: 4, 3: 8}[fcs_flag])
    if fcs_bytes == 0:
        return None
    p = 5 + (0 if single else 1) + (4 if did == 3 else did)
    if len(b) < p + fcs_bytes:
        raise ValueError("zstd frame header truncated")
    v = int.from_bytes(bytes(b[p:p + fcs_bytes]), "little")
    return v + 256 if fcs_bytes == 2 else v


class ZstdLaunch:
    """A set of zstd frames (and lowcard expansions) decoded by one
    bs_zstd_decode launch, then one bs_lut_expand launch for every lowcard entry.
    Every pointer is a device address; the caller keeps the memory alive until
    the launch has run (`keep` holds what this object allocates)."""

    def __init__(self, device):
        self.device = require_gpu(device)
        self.tasks: list[tuple[int, int, int, int, int]] = []
        self.expands: list[tuple[int, int, int, int, int, int]] = []
        self.keep: list = []
        self.out_len = None               # per-task decoded bytes (device int64), set by prepare()
        self._prepared = None

    def __len__(self) -> int:
        return len(self.tasks)

    def add_frame(self, src_ptr: int, src_len: int, dst_ptr: int, dst_len: int, xor_ptr: int = 0) -> None:
        """Frames at src decode to exactly dst_len bytes at dst; with xor_ptr,
        those bytes are XOR-ed with dst_len bytes there (a delta's base)."""
        self.tasks.append((src_ptr, src_len, dst_ptr, dst_len, xor_ptr))

    def add_lowcard(self, blob_ptr: int, host_blob, out_ptr: int, n_elem: int, item_bytes: int) -> None:
        """A lowcard blob (device copy at blob_ptr, host bytes host_blob) into
        n_elem elements of item_bytes bytes at out_ptr."""
        import torch
        lc = parse_lowcard(host_blob)
        if lc.n_elem != n_elem:
            raise ValueError(f"lowcard decode: index count mismatch {lc.n_elem} vs {n_elem}")
        if lc.item_bytes != item_bytes:
            raise ValueError(f"lowcard decode: byte count mismatch {lc.n_elem * lc.item_bytes} vs "
                             f"{n_elem * item_bytes}")
        if n_elem == 0:
            return
        idx = torch.empty(n_elem, dtype=torch.uint8, device=self.device)
        self.keep.append(idx)
        self.add_frame(blob_ptr + lc.idx_off, lc.idx_len, idx.data_ptr(), n_elem)
        self.expands.append((idx.data_ptr(), n_elem, blob_ptr + lc.lut_off, lc.n_unique, item_bytes, out_ptr))

    def prepare(self) -> None:
        """Build the device task arrays (once; later launches reuse them)."""
        import torch
        if getattr(self, "_prepared", None) is not None:
            return
        L = _native.lib()
        zst = None
        if self.tasks:
            t = np.array(self.tasks, dtype=np.uint64).view(ZSTD_TASK_DTYPE).reshape(-1)
            d_tasks = upload_bytes(t.view(np.uint8), self.device)
            wb = int(L.bs_zstd_work_bytes(len(self.tasks)))
            work = torch.empty(wb, dtype=torch.uint8, device=self.device)
            self.out_len = torch.empty(len(self.tasks), dtype=torch.int64, device=self.device)
            self.keep += [d_tasks, work, self.out_len]
            zst = (d_tasks, work, wb)
        luts = []
        if self.expands:
            t = np.zeros(len(self.expands), LUT_TASK_DTYPE)
            for i, (idx_ptr, n, lut_ptr, n_lut, ib, out_ptr) in enumerate(self.expands):
                t[i] = (idx_ptr, lut_ptr, out_ptr, n, n_lut, ib)
            for c in range(0, len(t), 65535):           # grid.y limit of one launch
                part = t[c:c + 65535]
                d_lut = upload_bytes(part.view(np.uint8), self.device)
                self.keep.append(d_lut)
                luts.append((d_lut, len(part), int(part["n"].max())))
        self._prepared = (zst, luts)

    def launch(self, status: StatusWord, stream=None) -> None:
        self.prepare()
        L = _native.lib()
        s = stream_ptr(stream, self.device)
        zst, luts = self._prepared
        if zst is not None:
            d_tasks, work, wb = zst
            _native.check(L.bs_zstd_decode(d_tasks.data_ptr(), len(self.tasks), work.data_ptr(), wb,
                                           self.out_len.data_ptr(), status.ptr, s), "bs_zstd_decode")
        for d_lut, n_tasks, max_n in luts:
            _native.check(L.bs_lut_expand(d_lut.data_ptr(), n_tasks, max_n, status.ptr, s), "bs_lut_expand")


def _decode_host_bytes(blob: bytes, n_bytes: int, lowcard_item_bytes: int = 0) -> bytes:
    import torch
    dev = require_gpu(None)
    d_blob = upload_bytes(np.frombuffer(blob, np.uint8), dev) if len(blob) else None
    out = torch.empty(max(n_bytes, 1), dtype=torch.uint8, device=dev)
    st = StatusWord(dev)
    z = ZstdLaunch(dev)
    if lowcard_item_bytes:
        if n_bytes % lowcard_item_bytes:
            raise ValueError(f"lowcard decode: {n_bytes} bytes is not a whole number of "
                             f"{lowcard_item_bytes}-byte elements")
        z.add_lowcard(d_blob.data_ptr() if d_blob is not None else 0, blob, out.data_ptr(),
                      n_bytes // lowcard_item_bytes, lowcard_item_bytes)
    else:
        if d_blob is None:
            raise ValueError("zstd decode: empty blob")
        z.add_frame(d_blob.data_ptr(), len(blob), out.data_ptr(), n_bytes)
    z.launch(st)
    torch.cuda.synchronize(dev)
    st.check("zstd decode")
    return out[:n_bytes].cpu().numpy().tobytes()


def decode_zstd(blob: bytes, extras: dict | None = None, n_bytes: int | None = None) -> bytes:
    """generic.decode_zstd (bigsmall/codecs/generic.py:15-18) on the GPU. The
    decoded size is n_bytes when given, else the frame's recorded content size."""
    if n_bytes is None:
        n_bytes = frame_content_size(blob)
        if n_bytes is None:
            raise ValueError("zstd frame does not record its content size; pass n_bytes")
    return _decode_host_bytes(bytes(blob), int(n_bytes))


def decode_lowcard(blob: bytes, extras: dict, n_bytes: int) -> bytes:
    """special.decode_lowcard (bigsmall/codecs/special.py:67-85) on the GPU."""
    if len(blob) < 1:
        raise ValueError("lowcard blob shorter than its 2-byte header")
    return _decode_host_bytes(bytes(blob), int(n_bytes), lowcard_item_bytes=max(1, blob[0]))


def decode_special(blob: bytes, extras: dict, n_bytes: int) -> bytes:
    """special.decode (bigsmall/codecs/special.py:150-156): lowcard only."""
    kind = (extras or {}).get("special_kind")
    if kind == "lowcard":
        return decode_lowcard(blob, extras, n_bytes)
    raise ValueError(f"Unknown special codec: {kind}")
