"""Per-tensor codec registry and auto-selection (mirrors bigsmall/codec_registry.py).

Plugin API, unchanged from the reference (codec_registry.py:39-55):
    register_codec(name, encode_fn, decode_fn); get_codec(name); registered_names()
    encode_fn(raw: bytes, **ctx) -> (blob, extras)
    decode_fn(blob: bytes, extras: dict, n_weights: int) -> bytes

Selection follows the reference's rules (codec_registry.py:210-398): try every
candidate of the tensor's format, keep the smallest blob, ties go to the
earliest candidate, a failing candidate is skipped, and the function never
raises (the last resort is `raw`). The candidates are the codecs this engine
can both encode and decode on the GPU. The reference's `prefer_speed` and
`enable_gpu_parallel` knobs are accepted: every candidate here is already a
GPU format, so they change nothing.
"""
from __future__ import annotations

from typing import Callable, Optional

from .codecs import bf16_chunked, bf16_parallel, bf16_tans, single_kernel, zstd_gpu

_REGISTRY: dict[str, tuple[Callable, Callable]] = {}


def register_codec(name: str, encode_fn: Callable, decode_fn: Callable) -> None:
    """Register a codec; overwrites any prior registration for `name`."""
    _REGISTRY[name] = (encode_fn, decode_fn)


def get_codec(name: str) -> Optional[tuple[Callable, Callable]]:
    return _REGISTRY.get(name)


def registered_names() -> list[str]:
    return list(_REGISTRY.keys())


def _enc_bf16_chunked(raw, **ctx):
    return bf16_chunked.encode(raw, **ctx)


def _enc_fp8_chunked(raw, **ctx):
    return bf16_chunked.encode_fp8(raw, **ctx)


def _enc_raw(raw, **_):
    return bytes(raw), {"n_bytes": len(raw)}


def _dec_raw(blob, extras, n_weights):
    return bytes(blob)


register_codec(bf16_chunked.CODEC_BF16, _enc_bf16_chunked, bf16_chunked.decode)
register_codec(bf16_chunked.CODEC_FP8, _enc_fp8_chunked, bf16_chunked.decode_fp8)
register_codec(bf16_parallel.CODEC, bf16_parallel.encode, bf16_parallel.decode)
register_codec(bf16_tans.CODEC, bf16_tans.encode, bf16_tans.decode)
register_codec(single_kernel.CODEC, single_kernel.encode, single_kernel.decode)
register_codec("raw", _enc_raw, _dec_raw)


def _enc_zstd_unavailable(raw, **_):
    raise NotImplementedError("this engine decodes zstd-coded entries; it does not write them")


def _dec_zstd(blob, extras, n_weights):
    """The reference registers zstd with generic.decode_zstd (codec_registry.py:171), which
    returns the frame's content whatever n_weights is; the size comes from the frame."""
    return zstd_gpu.decode_zstd(blob, extras)


register_codec("zstd", _enc_zstd_unavailable, _dec_zstd)

# Per-format ordered candidates. fp32/fp16 have no GPU codec here: they are
# stored raw (the reference's constriction codecs for them are not available).
CODEC_CANDIDATES: dict[str, list[str]] = {
    "bf16": [bf16_chunked.CODEC_BF16],
    "fp8": [bf16_chunked.CODEC_FP8],
    "fp32": ["raw"],
    "fp16": ["raw"],
    "fp4": ["raw"],
    "raw": ["raw"],
}


def auto_select_codec(raw: bytes, fmt: str, dtype: str, tensor_name: str = "", shape: tuple = (),
                      item_bytes: int = 0, prefer_speed: bool = False, enable_gpu_parallel: bool = False,
                      **_ignored) -> tuple[bytes, str, dict]:
    """Smallest blob over CODEC_CANDIDATES[fmt]; never raises (falls back to raw)."""
    best: Optional[tuple[bytes, str, dict]] = None
    for name in CODEC_CANDIDATES.get(fmt, ["raw"]):
        pair = _REGISTRY.get(name)
        if pair is None:
            continue
        try:
            blob, extras = pair[0](raw)
        except Exception:
            continue
        if best is None or len(blob) < len(best[0]):
            best = (blob, name, extras or {})
    if best is None:
        return bytes(raw), "raw", {"n_bytes": len(raw)}
    return best


class CodecStats:
    """Counts codec usage per run (codec_registry.py:401-413)."""

    __slots__ = ("counts",)

    def __init__(self) -> None:
        self.counts: dict[str, int] = {}

    def record(self, codec_name: str) -> None:
        self.counts[codec_name] = self.counts.get(codec_name, 0) + 1

    def as_dict(self) -> dict[str, int]:
        return dict(self.counts)
