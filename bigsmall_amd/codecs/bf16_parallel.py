"""`bf16_parallel_v1`: the reference's format, decoded on the GPU.

Same plugin shape as the reference (bigsmall/codecs/bf16_parallel.py:262-352):
    decode(blob: bytes, extras: dict, n_weights: int) -> bytes
The blob's framing is parsed on the host (bigsmall_amd/codecs/_refstreams.py);
every symbol is decoded by the HIP kernels behind bs_refcodec_decode. There is
no CPU decode path: without a ROCm GPU this raises.

encode(raw) writes the reference encoder's bytes (bigsmall/codecs/bf16_parallel.py:186-259) with this
library's host encoder (bs_refcodec_encode); compress() uses it for the
reference's gpu_optimised / prefer_speed choices.
"""
from __future__ import annotations

from . import _refstreams

CODEC = "bf16_parallel_v1"


def parse(blob: bytes, n_weights: int) -> _refstreams.RefPlan:
    """Host-side framing parse (raises ValueError on malformed blobs)."""
    return _refstreams.PARSERS[CODEC](bytes(blob), n_weights)


def decode(blob: bytes, extras: dict, n_weights: int) -> bytes:
    """Decode to raw bf16 bytes (little-endian), on the GPU."""
    return _refstreams.decode_host(CODEC, blob, n_weights)


def encode(raw: bytes, n_streams: int = 128, **_) -> tuple[bytes, dict]:
    """The reference's bf16_parallel.encode(raw, n_streams): N stride-interleaved
    rANS streams with shared tables; extras {"n_streams": N} as the reference's."""
    n = len(raw) // 2
    return _refstreams.encode_host(CODEC, raw, n_streams), {"n_streams": max(1, min(n_streams, n)) if n else n_streams}
