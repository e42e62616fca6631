"""Encoder: tensors -> .bs container in the engine's GPU format.

Mirrors the reference's `compress` (bigsmall/encoder.py:325-496): same header
fields per tensor (name, shape, dtype, codec, special, compressed_bytes,
offset, md5, extra) and per container (format, mode, model_type, base_model,
tensor_count, tensors, safetensors_metadata, codec_stats), the same routing
before codec selection (tensor_analysis.analyze_tensors, the reference's
tensor_analysis.py:80-132, restated in bigsmall_amd/tensor_analysis.py):
  * tied: a tensor byte-identical (md5) to an earlier one of the same shape and
    item size, at least 1024 bytes, becomes `tied_ref` (tensor_analysis.py:97-110);
  * tiny: fewer than RAW_TINY_THRESHOLD bytes are stored `raw` (encoder.py:57, 386-388);
  * everything else goes through codec_registry.auto_select_codec.
By default the codecs are bf16_chunked_v1 / fp8_chunked_v1 (GPU-native); the
reference's `lowcard` route for tensors with <= 16 distinct values is covered
by bf16_chunked_v1's exact-value mode, which codes up to 256 distinct values
per tensor and decodes in the same launch as its layer.
With gpu_optimised or prefer_speed the container holds only codecs the
reference decodes, routed as the reference routes them (encoder.py:140-189):
lowcard tensors (tensor_analysis.py:111-119) become `special` entries
(special.py:23-64, zstd through the system libzstd), bf16 tensors take
bf16_parallel_v1 / bf16_se_single_kernel / bf16_se_tans by
codec_registry.auto_select_reference_codec, anything else `zstd`. The
reference's wpe_delta route (blosc2, not installed here) is not taken: such
tensors go through the generic selection, as the reference's own encoder does
when that codec fails.
Blobs start on 256-byte boundaries of the data section (offsets are explicit
in the header, so any reader finds them).
"""
from __future__ import annotations

import hashlib
from pathlib import Path
from typing import Optional

import numpy as np

from . import codec_registry, container, formats, tensor_analysis
from .codecs import zstd_host

RAW_TINY_THRESHOLD = 512
TIE_MIN_BYTES = tensor_analysis.TIE_MIN_BYTES


def _tensor_record(name: str, t) -> dict:
    """name/shape/dtype/raw/fmt/item_bytes of a torch tensor (encoder.py:243-285)."""
    import torch
    t = t.detach().contiguous().cpu()
    dtype_str = str(t.dtype).replace("torch.", "")
    try:
        fmt = formats.detect_format_from_dtype(dtype_str)
    except ValueError:
        fmt = "raw"
    raw = t.view(torch.uint8).numpy().tobytes() if t.numel() else b""
    shape = list(t.shape)
    return {"name": name, "shape": shape, "dtype": dtype_str, "item_bytes": t.element_size(), "raw": raw,
            "fmt": fmt}


def _gather(src) -> tuple[list[dict], dict]:
    if isinstance(src, dict):
        return [_tensor_record(k, v) for k, v in src.items()], {}
    from safetensors import safe_open
    recs, meta = [], {}
    with safe_open(str(src), framework="pt") as f:
        try:
            meta = f.metadata() or {}
        except Exception:
            meta = {}
        for k in f.keys():
            recs.append(_tensor_record(k, f.get_tensor(k)))
    return recs, meta


def _detect_model_type(names: list[str]) -> str:
    """encoder.py:288-296."""
    blob = " ".join(names[:200]).lower()
    markers = ("unet", "vae", "controlnet", "double_block", "transformer_block", "x_embedder", "joint_blocks",
               "time_embed")
    return "diffusion" if any(m in blob for m in markers) else "llm"


def compress(src, dst: str | Path, mode: str = "balanced", workers: Optional[int] = None, progress: bool = False,
             exclude_names: Optional[set[str]] = None, enable_a5: bool = True, gpu_optimised: bool = False,
             prefer_speed: bool = False, steps: Optional[int] = None, **_ignored) -> str:
    """Compress a safetensors file (or a {name: torch.Tensor} dict) into a .bs container
    (bigsmall/encoder.py:325-496). gpu_optimised and prefer_speed select the
    reference's bf16_parallel_v1 / bf16_se_single_kernel / bf16_se_tans by its
    rules and write a container the reference itself reads (every entry in one
    of its codecs); `workers` is accepted for the reference's signature (the
    host encoders here thread internally)."""
    tensors, st_meta = _gather(src)
    if exclude_names:
        tensors = [t for t in tensors if t["name"] not in exclude_names]
    counts: dict[str, int] = {}
    for t in tensors:
        if t["fmt"] != "raw":
            counts[t["fmt"]] = counts.get(t["fmt"], 0) + 1
    dominant = max(counts, key=counts.get) if counts else "bf16"

    reference_readable = gpu_optimised or prefer_speed
    data = container.DataSectionBuilder()
    stats = codec_registry.CodecStats()
    header_tensors = []
    # md5 of every tensor up front, on a few threads (hashlib releases the GIL
    # on large buffers); the routing below uses them in tensor order
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(max(1, min(8, len(tensors)))) as pool:
        md5s = list(pool.map(lambda t: hashlib.md5(t["raw"]).hexdigest(), tensors))
    decisions, _ = tensor_analysis.analyze_tensors(tensors, md5s)
    for i, t in enumerate(tensors):
        raw = t["raw"]
        md5 = md5s[i]
        special = None
        kind = decisions[i]["kind"]
        if kind == "tied":
            blob, codec, extras = b"", "tied_ref", {"tied_to": tensors[decisions[i]["tied_to"]]["name"]}
            special = "tied"
        elif len(raw) < RAW_TINY_THRESHOLD:
            blob, codec, extras = raw, "raw", {"n_bytes": len(raw)}
        else:
            # wpe_delta takes the generic selection (its blosc2 coder is absent),
            # as the reference's encoder does when that coder fails (encoder.py:162-168)
            lowcard = reference_readable and kind == "lowcard"
            if lowcard:
                try:
                    blob, extras = zstd_host.encode_lowcard(raw, t["item_bytes"])
                    blob, codec, extras, special = blob, "special", {**extras, "special_kind": "lowcard"}, "lowcard"
                except (ValueError, RuntimeError):
                    lowcard = False                     # the generic selection, as the reference falls back
            if lowcard:
                pass
            elif reference_readable:
                blob, codec, extras = codec_registry.auto_select_reference_codec(
                    raw, t["fmt"], enable_gpu_parallel=gpu_optimised, prefer_speed=prefer_speed)
            elif steps is not None and t["fmt"] == "bf16":
                from .codecs import bf16_chunked
                blob, extras = bf16_chunked.encode(raw, steps=steps)
                codec = bf16_chunked.CODEC_BF16
            else:
                blob, codec, extras = codec_registry.auto_select_codec(
                    raw, t["fmt"], t["dtype"], t["name"], tuple(t["shape"]), t["item_bytes"], enable_a5=enable_a5,
                    enable_gpu_parallel=gpu_optimised, prefer_speed=prefer_speed)
            if codec == "bf16_parallel_v1":
                special = "gpu_parallel"                # the reference's label (encoder.py:185-186)
        off = data.add(blob)
        header_tensors.append({"name": t["name"], "shape": t["shape"], "dtype": t["dtype"], "codec": codec,
                               "special": special, "compressed_bytes": len(blob), "offset": off, "md5": md5,
                               "extra": extras or None})
        stats.record(codec)
    header = {"format": dominant, "mode": mode, "model_type": _detect_model_type([t["name"] for t in tensors]),
              "base_model": None, "tensor_count": len(tensors), "tensors": header_tensors,
              "safetensors_metadata": st_meta or None, "codec_stats": stats.as_dict()}
    # version 2 whenever a codec needs it (formats.V2_CODECS)
    version = formats.BS_FORMAT_VERSION_V2 if any(h["codec"] in formats.V2_CODECS for h in header_tensors) \
        else formats.BS_FORMAT_VERSION_V1
    container.write_container(dst, header, data.getvalue(), format_version=version)
    return str(dst)


def raw_words(t) -> np.ndarray:
    """bf16 tensor -> uint16 numpy view of its bit patterns (host)."""
    import torch
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
