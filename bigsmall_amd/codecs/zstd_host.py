"""Host-side zstd compression for containers written in the reference's own
codecs: the generic `zstd` codec (bigsmall/codecs/generic.py:9-12, level 9)
and the `special` lowcard codec (bigsmall/codecs/special.py:23-64: the sorted
distinct values and a level-19 zstd stream of one-byte indices).

The reference compresses with python-zstandard, which is not installed here;
this module calls the system libzstd through its C API (ZSTD_compress), which
writes the same kind of frame: content size in the header, no checksum. The
exact bytes of a frame depend on the zstd version, as the reference's do.
These entries decode on the GPU (codecs/zstd_gpu.py).
"""
from __future__ import annotations

import ctypes
import ctypes.util
import struct

import numpy as np

from .. import tensor_analysis

GENERIC_LEVEL = 9              # generic.encode_zstd default (generic.py:9)
LOWCARD_LEVEL = 19             # special.encode_lowcard (special.py:55)

_lib = None


def _load():
    global _lib
    if _lib is None:
        name = ctypes.util.find_library("zstd")
        if name is None:
            raise RuntimeError("zstd compression needs the system libzstd, which was not found")
        L = ctypes.CDLL(name)
        L.ZSTD_compressBound.restype = ctypes.c_size_t
        L.ZSTD_compressBound.argtypes = [ctypes.c_size_t]
        L.ZSTD_compress.restype = ctypes.c_size_t
        L.ZSTD_compress.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        L.ZSTD_isError.restype = ctypes.c_uint
        L.ZSTD_isError.argtypes = [ctypes.c_size_t]
        L.ZSTD_getErrorName.restype = ctypes.c_char_p
        L.ZSTD_getErrorName.argtypes = [ctypes.c_size_t]
        _lib = L
    return _lib


def available() -> bool:
    try:
        _load()
        return True
    except (RuntimeError, OSError):
        return False


def compress(data, level: int) -> bytes:
    """One zstd frame of `data` at `level`."""
    L = _load()
    src = np.frombuffer(bytes(data), np.uint8)
    cap = int(L.ZSTD_compressBound(src.size))
    dst = np.empty(max(cap, 1), np.uint8)
    n = L.ZSTD_compress(dst.ctypes.data, cap, src.ctypes.data if src.size else None, src.size, level)
    if L.ZSTD_isError(n):
        raise RuntimeError(f"ZSTD_compress: {L.ZSTD_getErrorName(n).decode()}")
    return dst[:n].tobytes()


def encode_zstd(raw, level: int = GENERIC_LEVEL, **_) -> tuple[bytes, dict]:
    """generic.encode_zstd (bigsmall/codecs/generic.py:9-12)."""
    return compress(raw, level), {"level": level, "n_bytes": len(raw)}


def _keys(raw, item_bytes: int) -> np.ndarray:
    if item_bytes not in (1, 2, 4):
        raise ValueError(f"Unsupported item_bytes={item_bytes}")
    return np.frombuffer(bytes(raw), dtype={1: "<u1", 2: "<u2", 4: "<u4"}[item_bytes])


# the lowcard test and its distinct-value count are the routing module's
# (tensor_analysis.py:37-51, 111-119 in the reference)
count_unique = tensor_analysis.distinct_values
is_lowcard = tensor_analysis.is_lowcard


def encode_lowcard(raw, item_bytes: int) -> tuple[bytes, dict]:
    """special.encode_lowcard (bigsmall/codecs/special.py:23-64): u8 item_bytes,
    u8 n_unique, the distinct values ascending (little-endian, item_bytes
    each), u32 length and the zstd frame of the u8 indices, u32 element count."""
    keys = _keys(raw, item_bytes)
    uniq, inverse = np.unique(keys, return_inverse=True)
    if len(uniq) > 255:
        raise ValueError(f"lowcard codec requires <= 255 unique values, got {len(uniq)}")
    idx = compress(inverse.astype(np.uint8).tobytes(), LOWCARD_LEVEL)
    blob = (struct.pack("<BB", item_bytes, len(uniq)) + uniq.astype(keys.dtype).tobytes() +
            struct.pack("<I", len(idx)) + idx + struct.pack("<I", keys.size))
    return blob, {"item_bytes": item_bytes, "n_unique": int(len(uniq))}
