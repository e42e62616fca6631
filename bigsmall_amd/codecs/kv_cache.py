"""KV-cache entry codec (mirrors bigsmall/codecs/kv_cache.py:41-117).

Entry layout, as in the reference (little-endian), K then V:
    [u8 version] then per tensor: [u8 ndim][i32 x ndim shape][u32 blob_len][blob]
Versions: 1 = bf16_se_ac blobs, 2 = bf16_se_rans blobs (both constriction
bitstreams, not decodable by this engine: BigSmallVersionError), 3 = this
engine's bf16_chunked_v1 blobs, decoded on the GPU.

Element count per tensor uses max(1, dim) like the reference (kv_cache.py:109-111).
"""
from __future__ import annotations

import struct

import numpy as np

from ..exceptions import BigSmallVersionError
from . import bf16_chunked

VERSION_GPU = 3
KV_STEPS = 256          # BSCK steps for KV blobs: a 256-token block of 8x128 heads is 8 chunks


def _tensor_words(t) -> tuple[np.ndarray, list[int]]:
    import torch
    if t.dtype != torch.bfloat16:
        raise ValueError(f"compress_kv_entry expects BF16 tensors, got {t.dtype}")
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1), list(t.shape)


def encode_words(words: np.ndarray, steps: int = KV_STEPS) -> bytes:
    return bf16_chunked.encode_array(words, steps=steps) if words.size else b""


def compress_kv_entry(keys, values) -> bytes:
    """Compress one K/V pair into a version-3 entry. Device tensors are encoded
    on the GPU and only the compressed bytes come back to the host; host
    tensors use the host encoder (the reference copies to the host and encodes
    there, kv_cache.py:28-38)."""
    import torch
    if keys.dtype != torch.bfloat16 or values.dtype != torch.bfloat16:
        raise ValueError("compress_kv_entry requires BF16 keys and values")
    gpu_blobs = None
    if keys.is_cuda and values.is_cuda and keys.numel() and values.numel():
        arena, spans = bf16_chunked.encode_device([keys, values], steps=KV_STEPS, compact=False)
        host = arena.cpu().numpy()
        gpu_blobs = [host[o:o + n].tobytes() for o, n in spans]
    out = bytearray(struct.pack("<B", VERSION_GPU))
    for i, t in enumerate((keys, values)):
        shape = list(t.shape)
        blob = gpu_blobs[i] if gpu_blobs is not None else encode_words(_tensor_words(t)[0])
        out += struct.pack("<B", len(shape))
        for s in shape:
            out += struct.pack("<i", int(s))
        out += struct.pack("<I", len(blob))
        out += blob
    return bytes(out)


def parse_kv_entry(data: bytes) -> list[tuple[list[int], int, int, int]]:
    """[(shape, n_elements, blob_offset, blob_len)] for K and V of an entry."""
    if not data:
        raise ValueError("empty KV entry")
    version = data[0]
    if version in (1, 2):
        from .. import __version__
        raise BigSmallVersionError(required="newer-than-installed", installed=__version__,
                                   detail=f"KV entry version {version} is constriction-coded; this engine "
                                          f"decodes version {VERSION_GPU}")
    if version != VERSION_GPU:
        raise ValueError(f"Unknown KV cache codec version {version}")
    pos, out = 1, []
    for _ in range(2):
        ndim = data[pos]
        pos += 1
        shape = list(struct.unpack_from(f"<{ndim}i", data, pos))
        pos += 4 * ndim
        blen, = struct.unpack_from("<I", data, pos)
        pos += 4
        if pos + blen > len(data):
            raise ValueError("KV entry truncated")
        n = 1
        for s in shape:
            n *= max(1, s)
        out.append((shape, n, pos, blen))
        pos += blen
    return out


def decompress_kv_entry(data: bytes, device: str = "cuda"):
    """Inverse of compress_kv_entry: (keys, values) as bf16 tensors on `device`."""
    import torch
    from ..device import ChunkBatch, ChunkJob, StatusWord, require_gpu, upload_bytes
    parts = parse_kv_entry(data)
    dev = require_gpu(device if str(device) != "cpu" else None)
    buf = np.zeros(sum(((b + 255) & ~255) for _, _, _, b in parts) + 256, np.uint8)
    jobs, outs, pos = [], [], 0
    for shape, n, off, blen in parts:
        buf[pos:pos + blen] = np.frombuffer(data, np.uint8, blen, off)
        outs.append((torch.empty(shape if all(s > 0 for s in shape) else [n], dtype=torch.bfloat16, device=dev),
                     pos, blen, n))
        pos += (blen + 255) & ~255
    d = upload_bytes(buf, dev)
    for o, p, blen, n in outs:
        if blen:
            inf = bf16_chunked.info(bytes(buf[p:p + 32]))
            if inf.n != n:
                raise ValueError(f"KV entry: blob holds {inf.n} elements, shape needs {n}")
            jobs.append(ChunkJob(d.data_ptr() + p, blen, o.data_ptr(), n, inf.n_chunks, inf.plane_mode))
    st = StatusWord(dev)
    if jobs:
        ChunkBatch(jobs, dev).launch(st)
    torch.cuda.synchronize(dev)
    st.check("KV entry")
    k, v = outs[0][0], outs[1][0]
    if str(device) == "cpu":
        return k.cpu(), v.cpu()
    return k, v
