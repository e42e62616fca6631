"""GPU backend of the decode engine (mirrors bigsmall/kernels/__init__.py:36-111).

    use_gpu() -> bool
    backend_name() -> "hip" | "cpu"
    decode_bf16_parallel(blob, extras, n_weights) -> bytes

One backend: the HIP kernels of libbigsmall_hip.so on a ROCm GPU (gfx950).
The reference probes CUDA-C, then Triton, and falls back to a CPU decoder
with a RuntimeWarning; this engine has no CPU decode path, so without a GPU
(or with BIGSMALL_FORCE_CPU=1, which the reference uses to disable the GPU)
decode_bf16_parallel raises RuntimeError instead of silently running elsewhere.
"""
from __future__ import annotations

import os
from typing import Optional

_GPU_BACKEND: Optional[str] = None   # None = not yet probed, "" = no GPU, "hip" otherwise


def _force_cpu() -> bool:
    return os.environ.get("BIGSMALL_FORCE_CPU", "").lower() in ("1", "true", "yes")


def _probe_backend() -> None:
    """Decide once whether the HIP backend is usable (cached like the reference's)."""
    global _GPU_BACKEND
    if _GPU_BACKEND is not None:
        return
    if _force_cpu():
        _GPU_BACKEND = ""
        return
    try:
        import torch
        if not torch.cuda.is_available():
            _GPU_BACKEND = ""
            return
        from .. import _native
        _native.lib()
        _GPU_BACKEND = "hip"
    except Exception:
        _GPU_BACKEND = ""


def use_gpu() -> bool:
    _probe_backend()
    return bool(_GPU_BACKEND)


def backend_name() -> str:
    """The backend's name: "hip", or "cpu" when no GPU backend is usable, the reference's names
    for the two cases (kernels/__init__.py:84-86), so callers that branch on
    them take the same branch. Here "cpu" means only that: there is no CPU
    decoder, and decode_bf16_parallel raises RuntimeError."""
    _probe_backend()
    return _GPU_BACKEND or "cpu"


def decode_bf16_parallel(blob: bytes, extras: dict, n_weights: int) -> bytes:
    """Decode a `bf16_parallel_v1` blob to raw BF16 bytes on the GPU."""
    if n_weights == 0 or len(blob) == 0:
        return b""
    if not use_gpu():
        raise RuntimeError("bigsmall_amd decodes on an AMD GPU; no usable ROCm device "
                           "(or BIGSMALL_FORCE_CPU is set) and there is no CPU decode path")
    from ..codecs import _refstreams
    return _refstreams.decode_host("bf16_parallel_v1", blob, n_weights)
