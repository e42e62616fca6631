"""ctypes binding of libbigsmall_hip.so (declarations: include/bigsmall_hip.h).

torch is imported before the library is loaded so the library binds to the
HIP runtime torch already mapped (one runtime per process: device pointers,
streams and events are shared with torch). The library must have been built
(`python -m bigsmall_amd.build` or __graft_entry__.build()); there is no
fallback: every decode entry point raises if it is missing.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("BIGSMALL_HIP_LIB") or Path(__file__).resolve().parent / "_lib" / "libbigsmall_hip.so")

BS_OK = 0
BS_ERR_ARG, BS_ERR_FORMAT, BS_ERR_CAP, BS_ERR_HIP, BS_ERR_COUNT = -1, -2, -3, -4, -5
BS_DEV_ERR_HEADER, BS_DEV_ERR_COUNT, BS_DEV_ERR_BOUNDS, BS_DEV_ERR_STREAM = 0x1, 0x2, 0x4, 0x8
BS_CHUNK_MODE_AUTO = -1

_ERR_NAMES = {
    BS_ERR_ARG: "bad argument", BS_ERR_FORMAT: "malformed blob header", BS_ERR_CAP: "capacity too small",
    BS_ERR_HIP: "HIP launch failure", BS_ERR_COUNT: "element count mismatch",
}


class NativeLibraryMissing(RuntimeError):
    pass


class BsChunkInfo(ctypes.Structure):
    _fields_ = [("n", ctypes.c_uint64), ("n_chunks", ctypes.c_uint32), ("steps", ctypes.c_uint32),
                ("lanes", ctypes.c_uint32), ("n_syms", ctypes.c_uint32), ("elem_bytes", ctypes.c_uint32),
                ("plane_mode", ctypes.c_uint32), ("coder", ctypes.c_uint32)]


# (restype, argtypes) of every symbol include/bigsmall_hip.h declares
_P, _U8P = ctypes.c_void_p, ctypes.c_void_p
_U32, _U64, _I32, _INT = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32, ctypes.c_int
SIGNATURES = {
    "bs_version": (_INT, []),
    "bs_chunk_inspect": (_INT, [_U8P, _U64, ctypes.POINTER(BsChunkInfo)]),
    "bs_chunk_chunks_per_group": (_INT, []),
    "bs_chunk_decode": (_INT, [_P, _U64, _P, _U64, _U32, _U32, _P, _P]),
    "bs_chunk_decode_batch": (_INT, [_P, _U32, _U32, _U32, _P, _P]),
    "bs_chunk_encode_bound": (_INT, [_U64, _U32, _U32, _U32, ctypes.POINTER(_U64)]),
    "bs_chunk_encode": (_INT, [_P, _U64, _U32, _U32, _U32, _I32, _P, _U64, ctypes.POINTER(_U64), _INT]),
    "bs_chunk_encode_bound_ex": (_INT, [_U64, _U32, _U32, _U32, _I32, ctypes.POINTER(_U64)]),
    "bs_chunk_encode_ex": (_INT, [_P, _U64, _U32, _U32, _U32, _I32, _I32, _P, _U64, ctypes.POINTER(_U64), _INT]),
    "bs_refcodec_decode": (_INT, [_P, _U32, _P, _P, _P, _U32, _P, _U32, _P, _U64, _P, _P, _P]),
    "bs_refcodec_serial_work_bytes": (_U64, [_U64, _U32]),
    "bs_chunk_encode_gpu_work_bytes": (_U64, [_U32, _U64, _U32]),
    "bs_chunk_encode_gpu": (_INT, [_P, _U32, _U32, _U32, _P, _U64, _P, _P, _P]),
    "bs_copy_spans": (_INT, [_P, _U32, _U64, _P, _P]),
    "bs_zstd_work_bytes": (_U64, [_U32]),
    "bs_zstd_decode": (_INT, [_P, _U32, _P, _U64, _P, _P, _P]),
    "bs_zstd_decode_static": (_INT, [_P, _U32, _P, _P, _P]),
    "bs_lut_expand": (_INT, [_P, _U32, _U64, _P, _P]),
    "bs_refcodec_decode_serial": (_INT, [_P, _U32, _P, _P, _P, _U32, _P, _U32, _P, _U64, _P, _U64, _P, _P]),
    "bs_refcodec_serial_tiles": (_U32, [_U64, _U32]),
    "bs_refcodec_encode_bound": (_U64, [_I32, _U64, _U32]),
    "bs_refcodec_encode": (_INT, [_I32, _P, _U64, _U32, _P, _U64, ctypes.POINTER(_U64), _INT]),
    "bs_refcodec_decode_serial_batch": (_INT, [_P, _U32, _U32, _U32, _U32, _U32, _P, _U64, _P, _P]),
    "bs_refcodec_serial_chains_per_group": (_U32, []),
}

_lib = None


def lib():
    """Load the library (once). Raises NativeLibraryMissing if it is not built."""
    global _lib
    if _lib is None:
        import torch  # noqa: F401  (bind to torch's HIP runtime)
        if not LIB_PATH.exists():
            raise NativeLibraryMissing(
                f"{LIB_PATH} is not built; run `python -m bigsmall_amd.build` (needs hipcc, gfx950)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != BS_OK:
        raise RuntimeError(f"{what}: {_ERR_NAMES.get(rc, 'error')} ({rc})")
