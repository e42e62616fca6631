"""Streaming loader: decode one transformer layer at a time into HBM.

Same interface as the reference's StreamingLoader (bigsmall/streaming.py:52-275):
`layer_index`, `tensor_names`, `layer_count`, `layer_tensor_names`,
`non_layer_tensor_names`, `load_tensor`, `load_layer`, `load_non_layer_tensors`,
`iter_layers`, context manager. A path is a single .bs file or a directory with
bigsmall.index.json (+ `duplicate_map` aliases, bigsmall/hub_index.py:186-202)
or plain *.bs shards.

Where the reference decodes each tensor on the CPU and copies it to the device
(streaming.py:163-191), a layer here is one GroupDecoder group: its compressed
span is read into pinned memory (in parallel pieces), copied host->device on a
copy stream and decoded by one batched kernel launch, on the loader's own
decode stream, straight into device tensors. With prefetch > 0 every
submission runs on one worker thread, so `iter_layers` (and
BigSmallStreamingModel) keep `prefetch` layers in flight: the file read, the
host->device copy and the decode of layer i+1 overlap the consumer's work on
layer i, which the caller queues on its own stream meanwhile. `collect` hands
the tensors to the caller's stream (GroupResult.wait).
"""
from __future__ import annotations

import json
import re
from concurrent.futures import Future, ThreadPoolExecutor
from pathlib import Path
from typing import Iterator, Optional

from . import container

_LAYER_RE = re.compile(r"(?:^|\.)(?:layers|h)\.(\d+)\.")
INDEX_FILENAME = "bigsmall.index.json"


def layer_index(name: str) -> Optional[int]:
    """Transformer layer index encoded in `name`, or None (bigsmall/streaming.py:30-38)."""
    m = _LAYER_RE.search(name)
    return int(m.group(1)) if m else None


class _TensorEntry:
    __slots__ = ("name", "meta", "shard_path", "data_offset")

    def __init__(self, name: str, meta: dict, shard_path: Path, data_offset: int):
        self.name, self.meta, self.shard_path, self.data_offset = name, meta, shard_path, data_offset


class StreamingLoader:
    """Decode a .bs model one transformer layer at a time.

    path: a .bs file, or a directory with bigsmall.index.json + shards (or *.bs).
    device: where the returned tensors live: a ROCm device ("cuda", "cuda:0",
        ...), or "cpu" (decoded on the GPU, then copied to host memory, as
        decoder.load does; the reference decodes on the CPU for it).
    dtype: optional torch dtype to cast floating tensors to.
    prefetch: layers decoded ahead by `iter_layers` (0 = decode on demand).
    """

    def __init__(self, path: str | Path, device: str = "cuda", dtype=None, prefetch: int = 1):
        self.device, self.dtype, self.path = device, dtype, Path(path)
        self._to_host = str(device).split(":")[0] == "cpu"
        self._decode_device = "cuda" if self._to_host else device
        self.prefetch = max(0, int(prefetch))
        self._index: dict[str, _TensorEntry] = {}
        self._layers: dict[int, list[str]] = {}
        self._non_layer: list[str] = []
        self._readers: dict[Path, object] = {}
        self._build_index()
        self._engine_obj = None
        self._worker: Optional[ThreadPoolExecutor] = None

    @property
    def _engine(self):
        # created on the first decode, so the index API works without a GPU;
        # its own decode stream lets a prefetched layer decode while the
        # caller's stream runs the current one
        if self._engine_obj is None:
            from . import engine
            self._engine_obj = engine.GroupDecoder(self._decode_device, stream="private",
                                                   n_pinned=max(2, self.prefetch + 1))
        return self._engine_obj

    def __enter__(self) -> "StreamingLoader":
        return self

    def __exit__(self, exc_type, exc, tb) -> None:
        self.close()

    def close(self) -> None:
        if self._worker is not None:
            self._worker.shutdown(wait=True)
            self._worker = None
        for r in self._readers.values():
            r.close()
        self._readers.clear()

    # ---------------------- index -------------------------------------------
    def _shards(self) -> tuple[list[Path], dict]:
        if self.path.is_dir():
            idx_file = self.path / INDEX_FILENAME
            if idx_file.exists():
                idx = json.loads(idx_file.read_text(encoding="utf-8"))
                meta = idx.get("metadata") or {}
                return [self.path / s for s in meta["shards"]], meta.get("duplicate_map") or {}
            shards = sorted(self.path.glob("*.bs"))
            if not shards:
                raise FileNotFoundError(f"No .bs files and no {INDEX_FILENAME} in {self.path}")
            return shards, {}
        if self.path.is_file():
            return [self.path], {}
        raise FileNotFoundError(f"Path not found: {self.path}")

    def _add(self, name: str, entry: _TensorEntry) -> None:
        self._index[name] = entry
        li = layer_index(name)
        if li is None:
            self._non_layer.append(name)
        else:
            self._layers.setdefault(li, []).append(name)

    def _build_index(self) -> None:
        """bigsmall/streaming.py:95-145."""
        shards, dup = self._shards()
        for shard in shards:
            header, data_offset = container.read_header(shard)
            for t in header["tensors"]:
                if t["name"] in self._index:
                    raise ValueError(f"Tensor {t['name']!r} appears in multiple shards "
                                     f"({self._index[t['name']].shard_path.name}, {shard.name})")
                self._add(t["name"], _TensorEntry(t["name"], t, shard, data_offset))
        for dup_name, info in dup.items():
            master = info.get("master") if isinstance(info, dict) else None
            if master in self._index and dup_name not in self._index:
                self._add(dup_name, self._index[master])

    # ---------------------- decode ------------------------------------------
    def _reader(self, shard: Path):
        from . import engine
        r = self._readers.get(shard)
        if r is None:
            r = self._readers[shard] = engine.file_span_reader(shard)
        return r

    def _master(self, entry: _TensorEntry, seen=None) -> _TensorEntry:
        """Follow tied_ref links to the entry holding the data (streaming.py:163-179)."""
        seen = set() if seen is None else seen
        while entry.meta["codec"] == "tied_ref":
            m = (entry.meta.get("extra") or {})["tied_to"]
            if m in seen:
                raise ValueError(f"Tied-ref cycle: {seen | {m}}")
            seen.add(entry.name)
            nxt = self._index.get(m)
            if nxt is None:
                raise KeyError(f"tied_ref master {m!r} not found in index")
            entry = nxt
        return entry

    def _submit_async(self, names: list[str]):
        """_submit on the worker thread (a Future), or inline without prefetch.
        Every submission takes this path, so the engine's pinned buffers and the
        file readers are only ever used by one thread at a time."""
        if self.prefetch == 0:
            return self._submit(names)
        if self._worker is None:
            self._worker = ThreadPoolExecutor(1, thread_name_prefix="bs-stream")
        return self._worker.submit(self._submit, names)

    def _submit(self, names: list[str]):
        """Start decoding `names` (asynchronously); returns [(GroupResult, {out name: master name})]."""
        import torch
        eng = self._engine
        with torch.cuda.device(eng.device):
            return self._submit_on(eng, names)

    def _submit_on(self, eng, names: list[str]):
        from . import engine
        by_shard: dict[Path, list] = {}
        alias: dict[str, str] = {}
        followers: dict[Path, list] = {}
        for n in names:
            own = self._index[n]
            e = self._master(own)
            lst = by_shard.setdefault(e.shard_path, [])
            if all(x.name != e.name for x in lst):
                lst.append(e)
            if n != e.name and (own.meta["dtype"] != e.meta["dtype"] or
                                [int(s) for s in own.meta["shape"]] != [int(s) for s in e.meta["shape"]]):
                # a follower of another dtype or shape: the engine reinterprets the
                # master's bytes for it before any dtype conversion
                followers.setdefault(e.shard_path, []).append(
                    {**own.meta, "name": n, "codec": "tied_ref", "extra": {"tied_to": e.name}})
                alias[n] = n
            else:
                alias[n] = e.name
        jobs = []
        for shard, ents in by_shard.items():
            metas = [e.meta for e in ents] + followers.get(shard, [])
            lo, hi = engine.group_span(metas)
            res = eng.decode_group(metas, self._reader(shard), lo, hi - lo, dtype=self.dtype)
            jobs.append(res)
        return jobs, alias

    def _collect(self, jobs, alias: dict) -> dict:
        decoded = {}
        for res in jobs:
            decoded.update(res.wait("streaming decode"))
        if self._to_host:
            decoded = {k: v.cpu() for k, v in decoded.items()}
        out = {}
        for n, m in alias.items():
            out[n] = decoded[m] if n == m else decoded[m].clone()
        return out

    # ---------------------- public API --------------------------------------
    def tensor_names(self) -> list[str]:
        return list(self._index.keys())

    def layer_count(self) -> int:
        return max(self._layers.keys()) + 1 if self._layers else 0

    def layer_tensor_names(self, layer_idx: int) -> list[str]:
        return list(self._layers.get(layer_idx, []))

    def non_layer_tensor_names(self) -> list[str]:
        return list(self._non_layer)

    def load_tensor(self, name: str):
        if name not in self._index:
            raise KeyError(f"Tensor {name!r} not in this BigSmall model")
        return self.collect(self._submit_async([name]))[name]

    def load_layer(self, layer_idx: int) -> dict:
        names = self._layers.get(layer_idx)
        if names is None:
            raise IndexError(f"Layer {layer_idx} not in this model (have {self.layer_count()} layers)")
        return self.collect(self._submit_async(names))

    def submit_layer(self, layer_idx: int):
        """Start decoding a layer; `collect(handle)` returns its tensors."""
        names = self._layers.get(layer_idx)
        if names is None:
            raise IndexError(f"Layer {layer_idx} not in this model (have {self.layer_count()} layers)")
        return self._submit_async(names)

    def collect(self, handle) -> dict:
        """The tensors of a submitted group, ready for use on the caller's current stream."""
        if isinstance(handle, Future):
            handle = handle.result()
        return self._collect(*handle)

    def load_non_layer_tensors(self) -> dict:
        if not self._non_layer:
            return {}
        return self.collect(self._submit_async(self._non_layer))

    def iter_layers(self, progress: bool = True) -> Iterator[tuple[int, dict]]:
        """Yield (layer_idx, tensors) in order; `prefetch` layers ahead are
        already being copied and decoded while the caller works."""
        order = sorted(self._layers)
        inflight: list = []
        nxt = 0
        for i in order:
            while nxt < len(order) and len(inflight) <= self.prefetch:
                inflight.append((order[nxt], self.submit_layer(order[nxt])))
                nxt += 1
            li, handle = inflight.pop(0)
            layer = self.collect(handle)
            try:
                yield li, layer
            finally:
                layer.clear()


def decompress_layers(bs_path: str | Path, layer_indices: list[int], *, device: str = "cpu", dtype=None,
                      include_non_layer: bool = False) -> dict:
    """Only the named transformer layers of a .bs file or shard directory
    (bigsmall/hub_streaming.py:121-160): {name: tensor} on `device`, plus the
    non-layer tensors when include_non_layer. A missing layer raises
    ValueError. Each layer is one batched decode on the GPU."""
    out: dict = {}
    with StreamingLoader(bs_path, device=device, dtype=dtype, prefetch=0) as loader:
        if include_non_layer:
            out.update(loader.load_non_layer_tensors())
        for li in layer_indices:
            try:
                out.update(loader.load_layer(li))
            except IndexError:
                raise ValueError(f"decompress_layers: layer {li} not present in this model "
                                 f"(have {loader.layer_count()} layers)") from None
    return out
