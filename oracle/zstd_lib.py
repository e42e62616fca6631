"""ORACLE — test infrastructure, not part of the product.

The reference compresses and decompresses its zstd-coded entries with the
`zstandard` package (zstandard>=0.21, setup.py:28; bigsmall/codecs/generic.py:9-18,
bigsmall/codecs/special.py:23-85), which is not installed here. Its algorithm
is the published Zstandard format (RFC 8878), and this module checks against
the system's reference implementation of that format, libzstd (1.4.8 in this
image), called through ctypes:
  - `decompress` is the oracle for the GPU decoder;
  - `compress` writes the frames the tests decode (any conforming frame must
    decode the same; frames written by another zstd version differ in bytes,
    not in meaning);
  - `encode_lowcard` / `encode_zstd` restate the reference's two encoders
    (special.py:23-64, generic.py:9-12) on top of `compress`.
"""
from __future__ import annotations

import ctypes
import ctypes.util
import io
import struct

import numpy as np

_MAGIC = b"\x28\xb5\x2f\xfd"


def _block(last: int, btype: int, size: int) -> bytes:
    return struct.pack("<I", last | (btype << 1) | (size << 3))[:3]


# Hand-built frames and what RFC 8878 3.1.1 says they decode to: an empty raw
# block, an RLE block, two raw blocks, a frame without a content size (window
# descriptor instead), and a skippable frame between two frames.
KNOWN_FRAMES = {
    "empty": (_MAGIC + b"\x20\x00" + _block(1, 0, 0), b""),
    "rle": (_MAGIC + b"\x20\x05" + _block(1, 1, 5) + b"a", b"aaaaa"),
    "raw2": (_MAGIC + b"\x20\x07" + _block(0, 0, 3) + b"abc" + _block(1, 0, 4) + b"defg", b"abcdefg"),
    "no_fcs": (_MAGIC + b"\x00\x50" + _block(1, 0, 2) + b"hi", b"hi"),
    "skippable": (_MAGIC + b"\x20\x01" + _block(1, 0, 1) + b"x" + b"\x5a\x2a\x4d\x18\x03\x00\x00\x00zzz"
                  + _MAGIC + b"\x20\x02" + _block(1, 1, 2) + b"y", b"xyy"),
}

_lib = None
# ZSTD_cParameter values (zstd.h, stable API since 1.4.0)
_C_LEVEL, _C_CONTENT_SIZE, _C_CHECKSUM = 100, 200, 201


def _zstd():
    global _lib
    if _lib is None:
        name = ctypes.util.find_library("zstd") or "libzstd.so.1"
        L = ctypes.CDLL(name)
        L.ZSTD_compressBound.restype = ctypes.c_size_t
        L.ZSTD_compressBound.argtypes = [ctypes.c_size_t]
        L.ZSTD_isError.restype = ctypes.c_uint
        L.ZSTD_isError.argtypes = [ctypes.c_size_t]
        L.ZSTD_createCCtx.restype = ctypes.c_void_p
        L.ZSTD_freeCCtx.argtypes = [ctypes.c_void_p]
        L.ZSTD_CCtx_setParameter.restype = ctypes.c_size_t
        L.ZSTD_CCtx_setParameter.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        L.ZSTD_compress2.restype = ctypes.c_size_t
        L.ZSTD_compress2.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                     ctypes.c_size_t]
        L.ZSTD_decompress.restype = ctypes.c_size_t
        L.ZSTD_decompress.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t]
        L.ZSTD_versionNumber.restype = ctypes.c_uint
        _lib = L
    return _lib


def available() -> bool:
    try:
        _zstd()
        return True
    except OSError:
        return False


def version() -> int:
    return int(_zstd().ZSTD_versionNumber())


def compress(data: bytes, level: int = 3, checksum: bool = False, content_size: bool = True) -> bytes:
    L = _zstd()
    data = bytes(data)
    cap = int(L.ZSTD_compressBound(len(data)))
    out = ctypes.create_string_buffer(cap)
    src = ctypes.create_string_buffer(data, len(data)) if data else None
    c = L.ZSTD_createCCtx()
    try:
        for p, v in ((_C_LEVEL, level), (_C_CONTENT_SIZE, int(content_size)), (_C_CHECKSUM, int(checksum))):
            if L.ZSTD_isError(L.ZSTD_CCtx_setParameter(c, p, v)):
                raise ValueError(f"ZSTD_CCtx_setParameter({p}, {v}) failed")
        r = L.ZSTD_compress2(c, out, cap, src, len(data))
    finally:
        L.ZSTD_freeCCtx(c)
    if L.ZSTD_isError(r):
        raise ValueError("ZSTD_compress2 failed")
    return out.raw[:r]


def decompress(frame: bytes, n_bytes: int) -> bytes:
    """All frames in `frame`, which must decode to exactly n_bytes."""
    L = _zstd()
    frame = bytes(frame)
    out = ctypes.create_string_buffer(max(n_bytes, 1))
    r = L.ZSTD_decompress(out, n_bytes, frame, len(frame))
    if L.ZSTD_isError(r) or r != n_bytes:
        raise ValueError("ZSTD_decompress failed")
    return out.raw[:n_bytes]


def encode_zstd(raw: bytes, level: int = 9) -> tuple[bytes, dict]:
    """generic.encode_zstd (bigsmall/codecs/generic.py:9-12)."""
    return compress(raw, level), {"level": level, "n_bytes": len(raw)}


def encode_lowcard(raw: bytes, item_bytes: int) -> tuple[bytes, dict]:
    """special.encode_lowcard (bigsmall/codecs/special.py:23-64): the sorted
    distinct element values (at most 256) and a level-19 zstd frame of one
    uint8 index per element, framed as [u8 item_bytes][u8 n_unique][values]
    [u32 frame length][frame][u32 element count]."""
    arr = np.frombuffer(raw, dtype=np.uint8).reshape(-1, item_bytes)
    keys = np.zeros(len(arr), np.uint64)
    for b in range(item_bytes):
        keys |= arr[:, b].astype(np.uint64) << np.uint64(8 * b)
    uniq, inverse = np.unique(keys, return_inverse=True)
    if len(uniq) > 256:
        raise ValueError(f"lowcard codec requires <= 256 unique values, got {len(uniq)}")
    values = np.zeros((len(uniq), item_bytes), np.uint8)
    for b in range(item_bytes):
        values[:, b] = (uniq >> np.uint64(8 * b)) & np.uint64(0xFF)
    frame = compress(inverse.astype(np.uint8).tobytes(), 19)
    out = io.BytesIO()
    out.write(struct.pack("<BB", item_bytes, len(uniq)))
    out.write(values.tobytes())
    out.write(struct.pack("<I", len(frame)))
    out.write(frame)
    out.write(struct.pack("<I", len(arr)))
    return out.getvalue(), {"item_bytes": item_bytes, "n_unique": len(uniq)}


def decode_lowcard(blob: bytes, n_bytes: int) -> bytes:
    """special.decode_lowcard (bigsmall/codecs/special.py:67-85) with libzstd."""
    inp = io.BytesIO(blob)
    ib, nu = struct.unpack("<BB", inp.read(2))
    values = np.frombuffer(inp.read(nu * ib), np.uint8).reshape(nu, ib)
    flen, = struct.unpack("<I", inp.read(4))
    frame = inp.read(flen)
    n_elem, = struct.unpack("<I", inp.read(4))
    idx = np.frombuffer(decompress(frame, n_elem), np.uint8)
    out = values[idx].reshape(-1)
    if out.nbytes != n_bytes:
        raise ValueError(f"lowcard decode: byte count mismatch {out.nbytes} vs {n_bytes}")
    return out.tobytes()
