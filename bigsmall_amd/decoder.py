"""BigSmall decoder: .bs container -> tensors, decoded on the GPU.

Same public functions as the reference (bigsmall/decoder.py):
    decompress(src, dst=None, progress=True) -> dict[str, np.ndarray]   (decoder.py:100-157)
    load(src, device="cuda", progress=True) -> dict[str, torch.Tensor]    (decoder.py:301-310)
    _decode_blob(t, blob) -> bytes | None                                 (decoder.py:49-97)
    _raw_to_numpy, _numpy_to_torch                                       (decoder.py:249-298)

Differences that follow from decoding on the device:
  * `load` never materialises decoded weights in host memory: the container's
    compressed bytes go to HBM (pinned, asynchronous, one transformer layer at
    a time so the copy of layer i+1 overlaps the decode of layer i) and the
    kernels write the bf16/fp8 tensors in place. `device` must be a ROCm GPU
    ("cpu" decodes on the GPU and copies the result to the host).
  * `decompress` is `load` followed by one device->host copy per tensor.
  * There is no CPU decode path: without a GPU these raise RuntimeError.
"""
from __future__ import annotations

from pathlib import Path
from typing import Optional

import numpy as np

from . import container, engine
from .codecs import _refstreams, bf16_chunked, zstd_gpu
from .formats import DTYPE_BYTES
from .streaming import layer_index

_DTYPE_TO_NUMPY = {
    "F32": np.float32, "float32": np.float32, "F16": np.float16, "float16": np.float16,
    "BF16": None, "bfloat16": None,          # numpy has no bf16: uint16 view
    "F8_E4M3": np.uint8, "float8_e4m3fn": np.uint8, "F8_E5M2": np.uint8, "float8_e5m2": np.uint8,
    "I64": np.int64, "int64": np.int64, "I32": np.int32, "int32": np.int32,
    "I16": np.int16, "int16": np.int16, "I8": np.int8, "int8": np.int8,
    "U8": np.uint8, "uint8": np.uint8, "BOOL": np.bool_, "bool": np.bool_,
}


def _decode_blob(t: dict, blob: bytes):
    """Decode one tensor blob to raw bytes (host bytes in and out; the decode
    runs on the GPU). `tied_ref` -> None (caller resolves), `raw` -> the blob,
    an unknown or unsupported codec -> BigSmallVersionError."""
    engine.check_supported(t)
    codec = t["codec"]
    n = engine.entry_numel(t)
    extras = t.get("extra") or {}
    if codec == "tied_ref":
        return None
    if codec == "raw":
        return blob
    if codec in engine.BSCK_CODECS:
        return bf16_chunked.decode(blob, extras, n, elem_bytes=engine.BSCK_CODECS[codec])
    if codec == "bf16_parallel_v1":
        from . import kernels
        return kernels.decode_bf16_parallel(blob, extras, n)
    if codec in engine.ZSTD_CODECS:                  # zstd_xor_delta: the XOR delta itself (decoder.py:88-90)
        ib = DTYPE_BYTES.get(t["dtype"])
        return zstd_gpu.decode_zstd(blob, extras, n * ib if ib else None)
    if codec == "special":
        return zstd_gpu.decode_special(blob, extras, n * int(extras.get("item_bytes", 1)))
    return _refstreams.decode_host(codec, blob, n)


def layer_groups(tensors: list[dict]) -> list[list[dict]]:
    """Container entries grouped for decoding: one group per transformer layer
    (names matched like bigsmall/streaming.py:30), non-layer entries one group
    each, in data-section order."""
    by_layer: dict[int, list[dict]] = {}
    groups: list[list[dict]] = []
    for t in tensors:
        li = layer_index(t["name"])
        if li is None:
            groups.append([t])
        elif li in by_layer:
            by_layer[li].append(t)
        else:
            by_layer[li] = [t]
            groups.append(by_layer[li])
    key = lambda g: min((int(t["offset"]) for t in g if t["codec"] != "tied_ref"), default=1 << 62)
    return sorted(groups, key=key)


def load_to_device(src, device="cuda", dtype=None, decoder: engine.GroupDecoder | None = None,
                   xor_base: Optional[dict] = None) -> dict:
    """Decode every tensor of a container into device tensors (header order).
    xor_base: base tensors (same device) for the zstd_xor_delta entries of a
    delta container, which then decode to base XOR delta."""
    src = Path(src)
    header, _ = container.read_header(src)
    tensors = header["tensors"]
    dec = decoder or engine.GroupDecoder(device)
    reader = engine.file_span_reader(src)
    decoded: dict = {}
    pending: list[engine.GroupResult] = []
    try:
        deferred = []
        for g in layer_groups(tensors):
            masters_elsewhere = [t for t in g if t["codec"] == "tied_ref"
                                 and (t.get("extra") or {}).get("tied_to") not in {x["name"] for x in g}]
            if masters_elsewhere:
                deferred.append(g)
                continue
            lo, hi = engine.group_span(g)
            res = dec.decode_group(g, reader, lo, hi - lo, xor_base=xor_base)
            pending.append(res)
            decoded.update(res.tensors)
        for res in pending:
            res.wait("decode")
        for g in deferred:        # groups holding ties to tensors of other groups
            lo, hi = engine.group_span(g)
            res = dec.decode_group(g, reader, lo, hi - lo, resolve_tied=decoded.get, xor_base=xor_base)
            decoded.update(res.wait("decode"))
    finally:
        reader.close()
    # dtype conversion after every tie is resolved: a follower takes its
    # master's stored bytes, never converted ones
    conv = lambda v: v.to(dtype) if dtype is not None and v.is_floating_point() and v.dtype != dtype else v
    return {t["name"]: conv(decoded[t["name"]]) for t in tensors}


def load(src: str | Path, device: str = "cuda", progress: bool = True) -> dict:
    """Decompress and return tensors as torch.Tensors on `device`
    (bigsmall/decoder.py:301-310)."""
    import torch
    dev = torch.device(device)
    if dev.type == "cpu":
        return {k: v.cpu() for k, v in load_to_device(src, "cuda").items()}
    return load_to_device(src, dev)


def _to_numpy(t, dtype_str: str, shape) -> np.ndarray:
    import torch
    a = t.detach().contiguous().cpu()
    if a.dtype in (torch.bfloat16, torch.float16) and _DTYPE_TO_NUMPY.get(dtype_str) is None:
        arr = a.view(torch.int16).numpy().view(np.uint16)
    elif a.element_size() == 1 and a.dtype not in (torch.uint8, torch.int8, torch.bool):
        arr = a.view(torch.uint8).numpy()
    else:
        arr = a.numpy()
    return arr.reshape(shape) if shape else arr.reshape(-1)


def decompress(src: str | Path, dst: Optional[str | Path] = None, progress: bool = True) -> dict:
    """Decompress a .bs file to {name: numpy array} (bigsmall/decoder.py:100-157).
    BF16 comes back as a uint16 view, fp8 as uint8, like the reference."""
    header, _ = container.read_header(Path(src))
    dev = load_to_device(src, "cuda")
    out = {t["name"]: _to_numpy(dev[t["name"]], t["dtype"], t["shape"]) for t in header["tensors"]}
    if dst is not None:
        _write_safetensors(dst, out, header)
    return out


def _load_base_device(base_src, device) -> dict:
    """Base tensors of a delta on `device`, from a .bs container (decoded by
    this engine) or a safetensors file (bigsmall/decoder.py:212-246)."""
    base_src = Path(base_src)
    if base_src.suffix == ".bs":
        return load_to_device(base_src, device)
    from safetensors import safe_open
    out = {}
    with safe_open(str(base_src), framework="pt") as f:
        for k in f.keys():
            out[k] = f.get_tensor(k).contiguous().to(device)
    return out


def load_delta(delta_src: str | Path, base_src: str | Path, device: str = "cuda") -> dict:
    """A fine-tune stored as a delta container, reconstructed on the GPU: the
    zstd_xor_delta entries decode and XOR with their base tensor in one
    kernel; other entries decode as in `load`. Returns device tensors."""
    import torch
    dev = torch.device(device)
    header, _ = container.read_header(Path(delta_src))
    base = _load_base_device(base_src, dev)
    xor = {}
    for t in header["tensors"]:
        if t["codec"] == "zstd_xor_delta":
            if t["name"] not in base:
                raise KeyError(t["name"])
            b = base[t["name"]]
            xor[t["name"]] = b.view(-1).view(torch.uint8) if b.numel() else b
    return load_to_device(delta_src, dev, xor_base=xor)


def decompress_delta(delta_src: str | Path, base_src: str | Path, dst: Optional[str | Path] = None,
                     progress: bool = True) -> dict:
    """Decompress a delta .bs file against its base (safetensors or .bs);
    returns {name: numpy array} like bigsmall/decoder.py:160-210. The base
    tensors go to the GPU, and every zstd_xor_delta entry is decoded and XOR-ed
    with its base there."""
    header, _ = container.read_header(Path(delta_src))
    dev = load_delta(delta_src, base_src, "cuda")
    out = {t["name"]: _to_numpy(dev[t["name"]], t["dtype"], t["shape"]) for t in header["tensors"]}
    if dst is not None:
        _write_safetensors(dst, out, header)
    return out


def _raw_to_numpy(raw: bytes, dtype_str: str, shape: list[int]) -> np.ndarray:
    """bigsmall/decoder.py:249-263."""
    np_dtype = _DTYPE_TO_NUMPY.get(dtype_str)
    if np_dtype is None:
        np_dtype = np.uint16
    arr = np.frombuffer(raw, dtype=np_dtype)
    if not shape:
        return arr
    return arr.reshape(shape)


def _numpy_to_torch(arr: np.ndarray, dtype_str: str):
    """bigsmall/decoder.py:280-298."""
    import torch
    if dtype_str in ("BF16", "bfloat16"):
        return torch.from_numpy(arr.astype(np.uint16, copy=False).copy()).view(torch.bfloat16)
    if dtype_str in ("F8_E4M3", "float8_e4m3fn"):
        return torch.from_numpy(arr.astype(np.uint8, copy=False).copy()).view(torch.float8_e4m3fn)
    if dtype_str in ("F8_E5M2", "float8_e5m2"):
        return torch.from_numpy(arr.astype(np.uint8, copy=False).copy()).view(torch.float8_e5m2)
    return torch.from_numpy(arr.copy())


def _write_safetensors(dst, tensors: dict, header: dict) -> None:
    from safetensors.torch import save_file
    save_file({t["name"]: _numpy_to_torch(tensors[t["name"]], t["dtype"]) for t in header["tensors"]}, str(dst))


__all__ = ["decompress", "decompress_delta", "load", "load_delta", "load_to_device", "layer_groups", "_decode_blob",
           "_raw_to_numpy", "_numpy_to_torch"]
