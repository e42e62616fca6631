"""Compressed KV-cache manager (mirrors bigsmall/kv_cache_manager.py:22-91).

Whole-entry API, as in the reference: set(layer_idx, keys, values),
get(layer_idx) -> (keys, values), has, memory_usage, raw_size,
compression_ratio, clear, len, repr. Entries are version-3 (bf16_chunked_v1)
and decode on the GPU.

Block API (the reference keys one blob per layer and has no blocks; this adds
them for on-the-fly attention over a long cache):
    set_blocks(layer_idx, keys, values, block_tokens=256, token_dim=-2)
        splits K and V along the token dimension into blocks, encodes every
        block (on the GPU when K and V are device tensors, else with the host
        encoder) and keeps the compressed blocks resident in HBM, one arena
        per layer;
    get_blocks(layer_idx, block_ids) -> (K, V) with shape [len(block_ids), *block_shape]
    get_blocks_multi([(layer_idx, block_ids), ...]) -> [(K, V), ...]
        decode every requested block of every request in ONE batched kernel
        launch straight into the output tensors.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from .codecs import bf16_chunked
from .codecs import kv_cache as _kv_codec


def _block_major(blocked, td: int):
    """blocked.movedim(td, 0).contiguous(): the block index first, every block
    contiguous. Copied as 8-byte words when the innermost dimension allows it
    (the same bytes in a quarter of the elements)."""
    import torch
    if (blocked.is_contiguous() and blocked.element_size() == 2 and blocked.shape[-1] % 4 == 0
            and blocked.storage_offset() % 4 == 0 and blocked.data_ptr() % 8 == 0):
        return blocked.view(torch.int64).movedim(td, 0).contiguous().view(blocked.dtype)
    return blocked.movedim(td, 0).contiguous()


@dataclass
class _LayerBlocks:
    """Compressed blocks of one layer: one device arena, per-block offsets."""
    block_shape: list
    block_elems: int
    arena: object                               # uint8 device tensor
    k_blocks: list = field(default_factory=list)  # (offset, nbytes, n_chunks, plane_mode)
    v_blocks: list = field(default_factory=list)


def _block_outputs(n_blocks: int, L, dev):
    """K and V outputs [n_blocks] + block_shape. The decoder writes each block
    at a 16-byte aligned address, so when a block is not a multiple of 8
    elements the blocks sit in a buffer with a padded stride (a strided view)."""
    import torch
    stride = (L.block_elems + 7) // 8 * 8
    if stride == L.block_elems:
        k = torch.empty([n_blocks] + L.block_shape, dtype=torch.bfloat16, device=dev)
        return k, torch.empty_like(k)
    inner = [int(np.prod(L.block_shape[d + 1:])) for d in range(len(L.block_shape))]
    outs = []
    for _ in range(2):
        buf = torch.empty(max(n_blocks, 1) * stride, dtype=torch.bfloat16, device=dev)
        outs.append(buf.as_strided([n_blocks] + L.block_shape, [stride] + inner))
    return outs[0], outs[1]


class CompressedKVCache:
    """Compressed KV storage. device: where get()/get_blocks() materialise tensors."""

    def __init__(self, device: str = "cuda"):
        self.device = device
        self._compressed: dict = {}
        self._raw_size_bytes = 0
        self._blocks: dict = {}
        self._block_raw = 0

    # ---- whole-entry API (reference semantics) ------------------------------
    def set(self, layer_idx, keys, values) -> None:
        import torch
        if keys.dtype != torch.bfloat16 or values.dtype != torch.bfloat16:
            raise ValueError("CompressedKVCache.set: keys and values must be BF16")
        raw = keys.element_size() * keys.numel() + values.element_size() * values.numel()
        self._compressed[layer_idx] = _kv_codec.compress_kv_entry(keys, values)
        self._raw_size_bytes += raw

    def get(self, layer_idx):
        if layer_idx not in self._compressed:
            raise KeyError(f"layer {layer_idx} not in CompressedKVCache")
        return _kv_codec.decompress_kv_entry(self._compressed[layer_idx], device=self.device)

    def has(self, layer_idx) -> bool:
        return layer_idx in self._compressed

    def memory_usage(self) -> int:
        blocks = sum(sum(b[1] for b in L.k_blocks) + sum(b[1] for b in L.v_blocks) for L in self._blocks.values())
        return sum(len(b) for b in self._compressed.values()) + blocks

    def raw_size(self) -> int:
        return self._raw_size_bytes + self._block_raw

    def compression_ratio(self) -> Optional[float]:
        raw = self.raw_size()
        return None if raw == 0 else self.memory_usage() / raw

    def clear(self) -> None:
        self._compressed.clear()
        self._blocks.clear()
        self._raw_size_bytes = self._block_raw = 0

    def __len__(self) -> int:
        # a layer stored through both set() and set_blocks() counts once
        return len(set(self._compressed) | set(self._blocks))

    def __repr__(self) -> str:
        cr = self.compression_ratio()
        return (f"CompressedKVCache(layers={len(self)} compressed={self.memory_usage() / 1e6:.2f}MB "
                f"raw={self.raw_size() / 1e6:.2f}MB ratio={f'{cr * 100:.2f}%' if cr is not None else 'n/a'})")

    # ---- block API ----------------------------------------------------------
    def set_blocks(self, layer_idx, keys, values, block_tokens: int = 256, token_dim: int = -2,
                   threads: Optional[int] = None) -> int:
        """Compress K and V of a layer in blocks of `block_tokens` tokens; returns the block count."""
        import torch
        from .device import require_gpu, upload_bytes
        if keys.dtype != torch.bfloat16 or values.dtype != torch.bfloat16 or keys.shape != values.shape:
            raise ValueError("set_blocks: keys and values must be BF16 tensors of one shape")
        td = token_dim % keys.dim()
        T = keys.shape[td]
        if T % block_tokens:
            raise ValueError(f"set_blocks: {T} tokens is not a multiple of block_tokens={block_tokens}")
        nb = T // block_tokens
        if layer_idx in self._blocks:          # replacing a layer: drop its raw size from the totals
            old = self._blocks.pop(layer_idx)
            self._block_raw -= 2 * 2 * old.block_elems * len(old.k_blocks)
        block_shape = list(keys.shape)
        block_shape[td] = block_tokens
        block_elems = int(np.prod(block_shape))
        if keys.is_cuda and values.is_cuda:
            # encode on the GPU: the blocks never leave HBM
            groups = []
            for t in (keys, values):
                shape = list(t.shape)
                pre, post = int(np.prod(shape[:td])), int(np.prod(shape[td + 1:]))
                seg_len = block_tokens * post
                if t.is_contiguous() and t.data_ptr() % 4 == 0 and seg_len % 512 == 0 and (T * post) % 8 == 0:
                    # read in place: block b is `pre` segments of block_tokens * post
                    # words, T * post words apart ([blocks, segments, seg_len])
                    groups.append(t.detach().view(pre, nb, seg_len).permute(1, 0, 2))
                else:
                    blocked = t.detach().reshape(shape[:td] + [nb, block_tokens] + shape[td + 1:])
                    groups.append(_block_major(blocked, td).reshape(nb, block_elems))
            if block_elems % 2 == 0:
                arena, offs, lens = bf16_chunked.encode_device_rows(groups, steps=_kv_codec.KV_STEPS)
            else:       # odd blocks are not 4-byte aligned rows: one task per block view
                arena, spans = bf16_chunked.encode_device([g[i] for g in groups for i in range(nb)],
                                                          steps=_kv_codec.KV_STEPS)
                offs, lens = np.array([o for o, _ in spans], np.int64), np.array([n for _, n in spans], np.int64)
            per = bf16_chunked.GPU_ENCODE_LANES * _kv_codec.KV_STEPS
            nch = (block_elems + per - 1) // per
            ent = [(off, ln, nch, bf16_chunked.MODE_DENSE) for off, ln in zip(offs.tolist(), lens.tolist())]
            self._blocks[layer_idx] = _LayerBlocks(block_shape, block_elems, arena, ent[:nb], ent[nb:])
            self._block_raw += 2 * keys.numel() * 2
            return nb
        blobs = {"k": [], "v": []}
        for which, t in (("k", keys), ("v", values)):
            # [..., T, ...] -> [nb, ..., block_tokens, ...] contiguous blocks
            shape = list(t.shape)
            blocked = t.detach().cpu().reshape(shape[:td] + [nb, block_tokens] + shape[td + 1:])
            blocked = blocked.movedim(td, 0).contiguous()
            words = blocked.view(torch.int16).numpy().view(np.uint16).reshape(nb, -1)
            blobs[which] = [_kv_codec.encode_words(words[i]) for i in range(nb)]
        sizes = [(len(b) + 255) & ~255 for b in blobs["k"] + blobs["v"]]
        arena_host = np.zeros(sum(sizes) + 256, np.uint8)
        entries = {"k": [], "v": []}
        pos = 0
        for which in ("k", "v"):
            for b in blobs[which]:
                arena_host[pos:pos + len(b)] = np.frombuffer(b, np.uint8)
                inf = bf16_chunked.info(b[:32])
                entries[which].append((pos, len(b), inf.n_chunks, inf.plane_mode))
                pos += (len(b) + 255) & ~255
        arena = upload_bytes(arena_host, require_gpu(self.device))
        self._blocks[layer_idx] = _LayerBlocks(block_shape, block_elems, arena, entries["k"], entries["v"])
        self._block_raw += 2 * keys.numel() * 2
        return nb

    def block_count(self, layer_idx) -> int:
        return len(self._blocks[layer_idx].k_blocks)

    def _block_ids(self, L: _LayerBlocks, layer_idx, block_ids) -> list[int]:
        """Block ids as ints, each in [0, block count): a negative id is an
        error, not a block counted from the end."""
        ids = [int(i) for i in block_ids]
        n = len(L.k_blocks)
        for bi in ids:
            if not 0 <= bi < n:
                raise IndexError(f"layer {layer_idx!r}: block {bi} out of range (layer has {n} blocks)")
        return ids

    def get_blocks(self, layer_idx, block_ids):
        return self.get_blocks_multi([(layer_idx, block_ids)])[0]

    def get_blocks_multi(self, requests, stream=None):
        """Decode the blocks of every (layer_idx, block_ids) request in one launch."""
        import torch
        from .device import ChunkBatch, ChunkJob, StatusWord, require_gpu
        dev = require_gpu(self.device)
        jobs, results = [], []
        for layer_idx, block_ids in requests:
            L = self._blocks[layer_idx]
            ids = self._block_ids(L, layer_idx, block_ids)
            k, v = _block_outputs(len(ids), L, dev)
            base = L.arena.data_ptr()
            for j, bi in enumerate(ids):
                for blocks, out in ((L.k_blocks, k), (L.v_blocks, v)):
                    off, nb, nch, mode = blocks[bi]
                    jobs.append(ChunkJob(base + off, nb, out[j].data_ptr(), L.block_elems, nch, mode))
            results.append((k, v))
        st = StatusWord(dev)
        if jobs:
            ChunkBatch(jobs, dev).launch(st, stream)
        torch.cuda.synchronize(dev)
        st.check("KV blocks")
        return [(k.contiguous(), v.contiguous()) for k, v in results]

    def prepare_blocks_multi(self, requests):
        """Allocate outputs and build the batched launch for `requests` once;
        returns (launch, outputs) where launch(status, stream) decodes again.
        Outputs are strided views when a block is not a multiple of 8 elements."""
        import torch
        from .device import ChunkBatch, ChunkJob, require_gpu
        dev = require_gpu(self.device)
        jobs, results = [], []
        for layer_idx, block_ids in requests:
            L = self._blocks[layer_idx]
            ids = self._block_ids(L, layer_idx, block_ids)
            k, v = _block_outputs(len(ids), L, dev)
            for j, bi in enumerate(ids):
                for blocks, out in ((L.k_blocks, k), (L.v_blocks, v)):
                    off, nb, nch, mode = blocks[bi]
                    jobs.append(ChunkJob(L.arena.data_ptr() + off, nb, out[j].data_ptr(), L.block_elems, nch, mode))
            results.append((k, v))
        return ChunkBatch(jobs, dev), results
