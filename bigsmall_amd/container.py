"""BigSmall .bs container reader/writer (layout of bigsmall/container.py:1-40).

    [4]  magic b"BGSM"
    [2]  u16 LE format version (1 or 2)
    [4]  u32 LE header-JSON length
    [N]  header JSON (utf-8)
    [..] data section: the tensors' blobs; tensor t's blob is
         data[t["offset"] : t["offset"] + t["compressed_bytes"]]

Same functions and semantics as the reference (write_container :59-82,
read_header :85-116, read_blob :119-124, info :170-268). This writer also
accepts an `align` so blobs start on 256-byte boundaries of the data section:
readers only use `offset`, so the padding is invisible to any reader, and the
GPU path can read every blob of an uploaded data section with aligned vector
loads.
"""
from __future__ import annotations

import json
import struct
from pathlib import Path
from typing import Any

from .exceptions import BigSmallVersionError
from .formats import BS_FORMAT_VERSION, BS_SUPPORTED_FORMAT_VERSIONS, DTYPE_BYTES

MAGIC = b"BGSM"
VERSION = BS_FORMAT_VERSION
BLOB_ALIGN = 256
__version__ = "3.12.0+mi355x"


def write_container(path, header: dict, data: bytes, format_version: int = BS_FORMAT_VERSION) -> None:
    """container.py:59-82."""
    if format_version not in BS_SUPPORTED_FORMAT_VERSIONS:
        raise ValueError(f"Unsupported BigSmall format version {format_version!r}; "
                         f"supported: {sorted(BS_SUPPORTED_FORMAT_VERSIONS)}")
    header_bytes = json.dumps(header, separators=(",", ":")).encode("utf-8")
    with open(path, "wb") as f:
        f.write(MAGIC)
        f.write(struct.pack("<H", format_version))
        f.write(struct.pack("<I", len(header_bytes)))
        f.write(header_bytes)
        f.write(data)


def read_header(path) -> tuple[dict, int]:
    """container.py:85-116: returns (header_dict, data_offset); header gains
    `_format_version`."""
    with open(path, "rb") as f:
        magic = f.read(4)
        if magic != MAGIC:
            raise ValueError(f"Not a BigSmall .bs file (magic={magic!r})")
        version, = struct.unpack("<H", f.read(2))
        if version not in BS_SUPPORTED_FORMAT_VERSIONS:
            raise BigSmallVersionError(
                required="2.4.0", installed=__version__,
                detail=(f"file uses container format v{version}; "
                        f"this engine supports {sorted(BS_SUPPORTED_FORMAT_VERSIONS)}"))
        header_len, = struct.unpack("<I", f.read(4))
        header_bytes = f.read(header_len)
        data_offset = f.tell()
    header = json.loads(header_bytes.decode("utf-8"))
    header["_format_version"] = version
    return header, data_offset


def read_blob(path, header: dict, data_offset: int, tensor_idx: int) -> bytes:
    """container.py:119-124."""
    t = header["tensors"][tensor_idx]
    with open(path, "rb") as f:
        f.seek(data_offset + t["offset"])
        return f.read(t["compressed_bytes"])


def tensor_numel(t: dict) -> int:
    n = 1
    for d in t["shape"]:
        n *= int(d)
    return n


def tensor_raw_bytes(t: dict) -> int:
    """container.py:_tensor_raw_bytes."""
    return int(tensor_numel(t) * DTYPE_BYTES.get(t["dtype"], 1))


class DataSectionBuilder:
    """Accumulates blobs at `align`-byte offsets (zero padding between blobs)."""

    def __init__(self, align: int = BLOB_ALIGN):
        self.align = align
        self.parts: list[bytes] = []
        self.size = 0

    def add(self, blob: bytes) -> int:
        pad = (-self.size) % self.align if blob else 0
        if pad:
            self.parts.append(b"\x00" * pad)
            self.size += pad
        off = self.size
        self.parts.append(blob)
        self.size += len(blob)
        return off

    def getvalue(self) -> bytes:
        return b"".join(self.parts)


def info(path) -> dict[str, Any]:
    """container.py:170-268 summary (no decompression)."""
    from .streaming import layer_index
    p = Path(path)
    header, data_offset = read_header(p)
    file_size = p.stat().st_size
    per_tensor, total_raw, fmt_break, special_counts = [], 0, {}, {}
    for t in header["tensors"]:
        raw_bytes = tensor_raw_bytes(t)
        total_raw += raw_bytes
        comp = int(t["compressed_bytes"])
        dt = t["dtype"]
        tf = ("bf16" if dt in ("BF16", "bfloat16") else "fp32" if dt in ("F32", "float32") else
              "fp16" if dt in ("F16", "float16") else "fp8" if "8" in dt and "F" in dt.upper() else "other")
        fmt_break[tf] = fmt_break.get(tf, 0) + 1
        sp = t.get("special")
        if sp:
            special_counts[sp] = special_counts.get(sp, 0) + 1
        per_tensor.append({"name": t["name"], "shape": t["shape"], "dtype": dt, "codec": t["codec"],
                           "special": sp, "raw_bytes": raw_bytes, "compressed_bytes": comp,
                           "ratio_pct": (comp / raw_bytes * 100.0) if raw_bytes else 0.0})
    non_layer_raw, layer_tot = 0, {}
    for pt in per_tensor:
        li = layer_index(pt["name"])
        if li is None:
            non_layer_raw += pt["raw_bytes"]
        else:
            layer_tot[li] = layer_tot.get(li, 0) + pt["raw_bytes"]
    largest = max(layer_tot.values()) if layer_tot else 0
    ranked = sorted([pt for pt in per_tensor if pt["compressed_bytes"] > 0 and pt["raw_bytes"] > 0],
                    key=lambda x: x["ratio_pct"])
    pick = lambda xs: [{k: x[k] for k in ("name", "ratio_pct", "raw_bytes", "compressed_bytes")} for x in xs]
    codec_stats = dict(header.get("codec_stats") or {})
    if not codec_stats:
        for pt in per_tensor:
            codec_stats[pt["codec"]] = codec_stats.get(pt["codec"], 0) + 1
    return {
        "path": str(p), "file_size": file_size, "data_offset": data_offset, "data_size": file_size - data_offset,
        "format": header.get("format"), "mode": header.get("mode", "balanced"),
        "model_type": header.get("model_type", "llm"), "base_model": header.get("base_model"),
        "tensor_count": header["tensor_count"], "estimated_raw_bytes": total_raw,
        "ratio_pct": (file_size / total_raw * 100) if total_raw else 0.0, "version": VERSION,
        "format_breakdown": fmt_break, "special_counts": special_counts, "codec_stats": codec_stats,
        "per_tensor": per_tensor, "top5_best": pick(ranked[:5]), "top5_worst": pick(ranked[-5:][::-1]),
        "layer_count": len(layer_tot), "non_layer_raw_bytes": non_layer_raw,
        "largest_layer_raw_bytes": largest, "streaming_peak_ram_bytes": non_layer_raw + largest,
    }
