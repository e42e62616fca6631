"""Per-tensor codec registry and auto-selection (mirrors bigsmall/codec_registry.py).

Plugin API, unchanged from the reference (codec_registry.py:39-55):
    register_codec(name, encode_fn, decode_fn); get_codec(name); registered_names()
    encode_fn(raw: bytes, **ctx) -> (blob, extras)
    decode_fn(blob: bytes, extras: dict, n_weights: int) -> bytes

auto_select_codec applies the reference's rules (codec_registry.py:210-398) to
whatever candidates and codecs are registered:
  * smallest blob over CODEC_CANDIDATES[fmt], ties to the earliest candidate,
    a failing candidate skipped (:283-309);
  * prefer_speed (bf16): bf16_se_single_kernel if within max(4 KB, 0.6 % of the
    raw size) of the best, else bf16_se_tans if within
    max(2 KB, prefer_speed_tolerance x raw) (:316-349);
  * a bf16_se_ac winner yields to bf16_se_rans within max(1 KB, 0.01 % of raw)
    (:356-370) (codecs a user may register; constriction is not bundled);
  * enable_gpu_parallel (bf16): bf16_parallel_v1 with gpu_parallel_n_streams
    streams if within gpu_parallel_tolerance of the best (:377-391);
  * the function never raises.
The bf16_sparsity_v1 / fp2_residual_v1 candidates of the reference's bf16 list
are tried only when registered (their coders are constriction's), under the
enable_a5 / enable_fp2_residual switches.

Differences, by construction of this engine: the default candidates are the
GPU-native formats (bf16_chunked_v1 / fp8_chunked_v1), and the last resort is
`raw` instead of zstd. One rule of its own: bf16_chunked_tans_v1, listed after
bf16_chunked_v1 (as in the default bf16 list), competes only against a
bf16_chunked_v1 winner in compact plane mode (a tensor of mostly exact values,
such as a pruned one), and wins when it is at most compact_tans_tolerance (1 %)
larger: compact chunks decode in 17-29 % less time under tANS (a half-pruned
8B layer: 0.131 against 0.185 ms, for 0.01 % more bytes). Elsewhere it is not
encoded (dense tensors decode at the same speed under either coder, and rANS
is smaller). A candidate list without it forces rANS, one with only it tANS. The reference formats it writes (bf16_parallel_v1,
bf16_se_tans, bf16_se_single_kernel) are byte-identical to the reference
encoder's.

auto_select_reference_codec picks only codecs the reference itself decodes,
for containers compress() writes with gpu_optimised or prefer_speed: the same
speed and GPU rules, measured against bf16_se_tans's size where the reference
measures against its constriction winner (bf16_se_rans / bf16_se_ac, order-0
coders of the same sign/exponent and mantissa symbols, which this engine
cannot write); when no rule picks a faster format it writes bf16_se_tans, and
every other format as zstd (the last entry of each reference candidate list).
"""
from __future__ import annotations

from typing import Callable, Optional

from .codecs import bf16_chunked, bf16_parallel, bf16_tans, single_kernel, zstd_gpu, zstd_host

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
# the same format with the tANS coder: forced by a CODEC_CANDIDATES override, as
# the reference forces its codecs (tests/test_b4_auto_select.py:121-132 there)
register_codec(bf16_chunked.CODEC_BF16_TANS, lambda raw, **ctx: bf16_chunked.encode_tans(raw, **ctx),
               bf16_chunked.decode)
register_codec(bf16_chunked.CODEC_FP8_TANS, lambda raw, **ctx: bf16_chunked.encode_fp8_tans(raw, **ctx),
               bf16_chunked.decode_fp8)
register_codec(bf16_parallel.CODEC, bf16_parallel.encode, bf16_parallel.decode)
register_codec(bf16_tans.CODEC, bf16_tans.encode, bf16_tans.decode)
register_codec(single_kernel.CODEC, single_kernel.encode, single_kernel.decode)
register_codec("raw", _enc_raw, _dec_raw)


def _enc_zstd(raw, **_):
    """generic.encode_zstd (bigsmall/codecs/generic.py:9-12) through the system libzstd."""
    return zstd_host.encode_zstd(raw)


def _dec_zstd(blob, extras, n_weights):
    """The reference registers zstd with generic.decode_zstd (codec_registry.py:171), which
    returns the frame's content whatever n_weights is; the size comes from the frame."""
    return zstd_gpu.decode_zstd(blob, extras)


register_codec("zstd", _enc_zstd, _dec_zstd)

# Per-format ordered candidates. fp32/fp16 have no GPU codec here: they are
# stored raw (the reference's constriction codecs for them are not available).
CODEC_CANDIDATES: dict[str, list[str]] = {
    "bf16": [bf16_chunked.CODEC_BF16, bf16_chunked.CODEC_BF16_TANS],
    "fp8": [bf16_chunked.CODEC_FP8],
    "fp32": ["raw"],
    "fp16": ["raw"],
    "fp4": ["raw"],
    "raw": ["raw"],
}


def _try(name: str, raw, **ctx):
    """(blob, extras) of a registered codec, or None when it is missing or raises."""
    pair = _REGISTRY.get(name)
    if pair is None:
        return None
    try:
        blob, extras = pair[0](raw, **ctx)
    except Exception:
        return None
    return blob, extras or {}


def auto_select_codec(raw: bytes, fmt: str, dtype: str, tensor_name: str = "", shape: tuple = (),
                      item_bytes: int = 0, enable_a5: bool = True, enable_fp2_residual: bool = True,
                      enable_gpu_parallel: bool = False, gpu_parallel_n_streams: int = 128,
                      gpu_parallel_tolerance: float = 0.01, prefer_speed: bool = False,
                      prefer_speed_tolerance: float = 0.0015, compact_tans_tolerance: float = 0.01,
                      **_ignored) -> tuple[bytes, str, dict]:
    """(blob, codec name, extras) chosen by the reference's rules (codec_registry.py:210-398),
    plus this engine's compact-tANS rule (module docstring)."""
    candidates = CODEC_CANDIDATES.get(fmt, ["raw"])
    best: Optional[tuple[bytes, str, dict]] = None
    for name in candidates:
        if name == "bf16_sparsity_v1" and not enable_a5:
            continue
        if name == "fp2_residual_v1" and not enable_fp2_residual:
            continue
        if name == bf16_chunked.CODEC_BF16_TANS and best is not None and best[1] == bf16_chunked.CODEC_BF16:
            # the compact-tANS rule (module docstring)
            if bf16_chunked.info(best[0]).plane_mode == bf16_chunked.MODE_COMPACT:
                got = _try(name, raw)
                if got is not None and len(got[0]) <= len(best[0]) * (1.0 + compact_tans_tolerance):
                    best = (got[0], name, got[1])
            continue
        got = _try(name, raw)
        if got is not None and (best is None or len(got[0]) < len(best[0])):
            best = (got[0], name, got[1])

    if prefer_speed and fmt == "bf16" and "bf16_se_tans" not in candidates and best is not None:
        sk = _try("bf16_se_single_kernel", raw)
        if sk is not None and len(sk[0]) <= len(best[0]) + max(4096, int(len(raw) * 0.006)):
            best = (sk[0], "bf16_se_single_kernel", sk[1])
        else:
            tans = _try("bf16_se_tans", raw)
            if tans is not None and len(tans[0]) <= len(best[0]) + max(2048, int(len(raw) * prefer_speed_tolerance)):
                best = (tans[0], "bf16_se_tans", tans[1])

    if fmt == "bf16" and best is not None and best[1] == "bf16_se_ac" and "bf16_se_rans" in candidates:
        r = _try("bf16_se_rans", raw)
        if r is not None and len(r[0]) - len(best[0]) <= max(1024, int(len(raw) * 0.0001)):
            best = (r[0], "bf16_se_rans", r[1])

    if enable_gpu_parallel and fmt == "bf16" and best is not None:
        par = _try("bf16_parallel_v1", raw, n_streams=gpu_parallel_n_streams)
        if par is not None and len(par[0]) <= int(len(best[0]) * (1.0 + gpu_parallel_tolerance)):
            best = (par[0], "bf16_parallel_v1", par[1])

    if best is None:
        return bytes(raw), "raw", {"n_bytes": len(raw)}
    return best


def auto_select_reference_codec(raw: bytes, fmt: str, enable_gpu_parallel: bool = False,
                                gpu_parallel_n_streams: int = 128, gpu_parallel_tolerance: float = 0.01,
                                prefer_speed: bool = False, prefer_speed_tolerance: float = 0.0015,
                                **_ignored) -> tuple[bytes, str, dict]:
    """(blob, codec name, extras) among the codecs the reference decodes, by the
    rules of codec_registry.py:316-349 (prefer_speed) and :377-391 (GPU
    parallel), applied in that order to a running best. prefer_speed's second
    rule (bf16_se_tans within a tolerance of the best) holds by construction:
    bf16_se_tans is the starting best."""
    if fmt == "bf16":
        best = _try("bf16_se_tans", raw)   # the stand-in for the reference's smallest candidate
        if best is not None:
            best = (best[0], "bf16_se_tans", best[1])
            if prefer_speed:
                sk = _try("bf16_se_single_kernel", raw)
                if sk is not None and len(sk[0]) <= len(best[0]) + max(4096, int(len(raw) * 0.006)):
                    best = (sk[0], "bf16_se_single_kernel", sk[1])
            if enable_gpu_parallel:
                par = _try("bf16_parallel_v1", raw, n_streams=gpu_parallel_n_streams)
                if par is not None and len(par[0]) <= int(len(best[0]) * (1.0 + gpu_parallel_tolerance)):
                    best = (par[0], "bf16_parallel_v1", par[1])
            return best
    z = _try("zstd", raw)
    if z is not None:
        return z[0], "zstd", z[1]
    return bytes(raw), "raw", {"n_bytes": len(raw)}


class CodecStats:
    """Counts codec usage per run (codec_registry.py:401-413)."""

    __slots__ = ("counts",)

    def __init__(self) -> None:
        self.counts: dict[str, int] = {}

    def record(self, codec_name: str) -> None:
        self.counts[codec_name] = self.counts.get(codec_name, 0) + 1

    def as_dict(self) -> dict[str, int]:
        return dict(self.counts)
