"""ctypes binding of the oracle C library (oracle/bs_oracle.c).

ORACLE — test infrastructure only (see oracle/__init__.py). Each wrapper names
the reference function it restates; the C file carries the file:line citations.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "_build" / "liboracle.so"

__all__ = [
    "build", "lib", "quantise_ref", "quantise_sk", "rans_encode", "rans_decode", "rans_decode_nb",
    "par1_encode", "par1_decode", "tans_encode", "tans_decode", "sk_encode", "sk_decode",
    "chunk_decode", "tans_table", "par1_decode_threads", "chunk_decode_threads", "OracleError",
]


class OracleError(RuntimeError):
    def __init__(self, where: str, code: int):
        super().__init__(f"oracle {where} failed with status {code}")
        self.code = code


def build(force: bool = False) -> Path:
    """Compile oracle/bs_oracle.c with the committed Makefile."""
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < (_HERE / "bs_oracle.c").stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(_HERE), "-B" if force else "all"], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P, S, I, I64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int64
        U32 = ctypes.c_uint32
        sig = {
            "orc_quantise_ref": (I, [P, I, U32, P]),
            "orc_quantise_sk": (I, [P, I, U32, P]),
            "orc_rans_encode": (I64, [P, S, P, I, U32, P, S]),
            "orc_rans_decode": (I, [P, S, S, P, I, U32, P]),
            "orc_rans_decode_nb": (I, [P, S, S, P, I, I, P]),
            "orc_par1_encode": (I64, [P, S, I, P, S]),
            "orc_par1_decode": (I, [P, S, S, P]),
            "orc_tans_encode": (I64, [P, S, P, S]),
            "orc_tans_decode": (I, [P, S, S, P]),
            "orc_sk_encode": (I64, [P, S, P, S]),
            "orc_sk_decode": (I, [P, S, S, P]),
            "orc_chunk_decode": (I, [P, S, S, P]),
            "orc_chunk_decode_range": (I, [P, S, S, P, S, S]),
            "orc_par1_decode_streams": (I, [P, S, S, P, S, S]),
            "orc_tans_table": (I, [P, I, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _u16(words) -> np.ndarray:
    if isinstance(words, (bytes, bytearray, memoryview)):
        return np.frombuffer(bytes(words), dtype="<u2").copy()
    return np.ascontiguousarray(words, dtype=np.uint16)


def quantise_ref(counts, M: int) -> np.ndarray:
    """rans.quantise_frequencies (bigsmall/codecs/rans.py:34-92)."""
    c = np.ascontiguousarray(counts, dtype=np.int64)
    out = np.zeros(len(c), np.uint32)
    rc = lib().orc_quantise_ref(_p(c), len(c), M, _p(out))
    if rc:
        raise OracleError("quantise_ref", rc)
    return out


def quantise_sk(counts, M: int) -> np.ndarray:
    """single_kernel._quantise_inplace (bigsmall/codecs/single_kernel.py:53-110)."""
    c = np.ascontiguousarray(counts, dtype=np.int64)
    out = np.zeros(len(c), np.uint32)
    rc = lib().orc_quantise_sk(_p(c), len(c), M, _p(out))
    if rc:
        raise OracleError("quantise_sk", rc)
    return out


def rans_encode(symbols, freqs, M: int) -> bytes:
    """rans.encode_stream (bigsmall/codecs/rans.py:115-162)."""
    s = np.ascontiguousarray(symbols, dtype=np.int32)
    f = np.ascontiguousarray(freqs, dtype=np.uint32)
    cap = 4 + 2 * len(s) + 16
    out = np.zeros(cap, np.uint8)
    n = lib().orc_rans_encode(_p(s), len(s), _p(f), len(f), M, _p(out), cap)
    if n < 0:
        raise OracleError("rans_encode", n)
    return out[:n].tobytes()


def rans_decode(data: bytes, n: int, freqs, M: int) -> np.ndarray:
    """rans.decode_stream (bigsmall/codecs/rans.py:165-207)."""
    d = np.frombuffer(bytes(data), np.uint8).copy()
    f = np.ascontiguousarray(freqs, dtype=np.uint32)
    out = np.zeros(max(n, 1), np.uint32)
    rc = lib().orc_rans_decode(_p(d), len(d), n, _p(f), len(f), M, _p(out))
    if rc:
        raise OracleError("rans_decode", rc)
    return out[:n]


def rans_decode_nb(data: bytes, n: int, freqs, precision: int) -> np.ndarray:
    """numba_rans.decode_stream (bigsmall/codecs/numba_rans.py:195-217)."""
    d = np.frombuffer(bytes(data), np.uint8).copy()
    f = np.ascontiguousarray(freqs, dtype=np.uint32)
    out = np.zeros(max(n, 1), np.uint32)
    rc = lib().orc_rans_decode_nb(_p(d), len(d), n, _p(f), len(f), precision, _p(out))
    if rc:
        raise OracleError("rans_decode_nb", rc)
    return out[:n]


def _encode(fn: str, words, cap: int, *extra) -> bytes:
    w = _u16(words)
    out = np.zeros(cap, np.uint8)
    n = getattr(lib(), fn)(_p(w), len(w), *extra, _p(out), cap)
    if n < 0:
        raise OracleError(fn, n)
    return out[:n].tobytes()


def _decode(fn: str, blob: bytes, n: int, itemsize: int = 2) -> bytes:
    b = np.frombuffer(bytes(blob), np.uint8).copy()
    out = np.zeros(max(n, 1) * itemsize, np.uint8)
    rc = getattr(lib(), fn)(_p(b), len(b), n, _p(out))
    if rc:
        raise OracleError(fn, rc)
    return out[: n * itemsize].tobytes()


def _cap(n: int) -> int:
    return 4 * n + 64 * 1024


def par1_encode(words, n_streams: int = 128) -> bytes:
    """bf16_parallel.encode (bigsmall/codecs/bf16_parallel.py:186-259)."""
    w = _u16(words)
    # per stream: its lengths, up to 256 exponents and their bucket fields
    return _encode("orc_par1_encode", w, _cap(len(w)) + 4096 * (n_streams + 1), n_streams)


def par1_decode(blob: bytes, n: int) -> bytes:
    """bf16_parallel.decode (bigsmall/codecs/bf16_parallel.py:262-352)."""
    return _decode("orc_par1_decode", blob, n)


def tans_encode(words) -> bytes:
    """bf16_tans.encode (bigsmall/codecs/bf16_tans.py:68-118)."""
    w = _u16(words)
    return _encode("orc_tans_encode", w, _cap(len(w)))


def tans_decode(blob: bytes, n: int) -> bytes:
    """bf16_tans.decode (bigsmall/codecs/bf16_tans.py:121-167)."""
    return _decode("orc_tans_decode", blob, n)


def sk_encode(words) -> bytes:
    """single_kernel.encode (bigsmall/codecs/single_kernel.py:586-600)."""
    w = _u16(words)
    return _encode("orc_sk_encode", w, _cap(len(w)))


def sk_decode(blob: bytes, n: int) -> bytes:
    """single_kernel.decode (bigsmall/codecs/single_kernel.py:603-613)."""
    return _decode("orc_sk_decode", blob, n)


def chunk_decode(blob: bytes, n: int, elem_bytes: int = 2) -> bytes:
    """CPU decode of the build's GPU-native BSCK format, either coder, layout
    versions 2 and 3 (no reference counterpart)."""
    return _decode("orc_chunk_decode", blob, n, elem_bytes)


def _threaded(fn: str, blob: bytes, n: int, itemsize: int, units: int, threads: int) -> bytes:
    """Decode with `threads` host threads, each taking a contiguous range of
    the blob's independent units (streams or chunks) into one shared output;
    the C calls run without the GIL."""
    from concurrent.futures import ThreadPoolExecutor
    b = np.frombuffer(bytes(blob), np.uint8).copy()
    out = np.zeros(max(n, 1) * itemsize, np.uint8)
    threads = max(1, min(threads, units))
    cuts = [units * i // threads for i in range(threads + 1)]
    f = getattr(lib(), fn)
    with ThreadPoolExecutor(threads) as ex:
        rcs = list(ex.map(lambda i: f(_p(b), len(b), n, _p(out), cuts[i], cuts[i + 1]), range(threads)))
    for rc in rcs:
        if rc:
            raise OracleError(fn, rc)
    return out[: n * itemsize].tobytes()


def par1_decode_threads(blob: bytes, n: int, threads: int) -> bytes:
    """bf16_parallel.decode with its N streams split over host threads (the
    streams are independent: bigsmall/codecs/bf16_parallel.py:298-351 decodes
    them one after another)."""
    n_streams = int.from_bytes(bytes(blob[8:10]), "little") if len(blob) >= 10 else 1
    return _threaded("orc_par1_decode_streams", blob, n, 2, max(1, n_streams), threads)


def chunk_decode_threads(blob: bytes, n: int, threads: int, elem_bytes: int = 2) -> bytes:
    """chunk_decode with the blob's chunks split over host threads."""
    n_chunks = int.from_bytes(bytes(blob[24:28]), "little") if len(blob) >= 28 else 1
    return _threaded("orc_chunk_decode_range", blob, n, elem_bytes, max(1, n_chunks), threads)


def tans_table(freqs) -> np.ndarray:
    """The BSCK tANS decode table (4096 uint32 entries) of quantised
    frequencies summing to 4096."""
    f = np.ascontiguousarray(freqs, dtype=np.uint32)
    out = np.zeros(4096, np.uint32)
    rc = lib().orc_tans_table(_p(f), len(f), _p(out))
    if rc != 0:
        raise OracleError("orc_tans_table", rc)
    return out
