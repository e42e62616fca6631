"""Local multi-shard models (the file side of bigsmall/hub.py:46-588).

`compress_for_hub(source_dir, output_dir)` turns a directory of safetensors
shards into .bs shards (`model.bs`, or `model-00001-of-0000N.bs`), stores
tensors that repeat across shards once (md5 + shape + dtype, >= 1024 bytes;
the aliases go to the index's `duplicate_map`), and writes
`bigsmall.index.json` (+ `bigsmall.index.bin` from 100 tensors on) and the
model's config/tokenizer files. `from_pretrained(path)` loads a .bs file or
such a directory into one state dict, decoding every shard on the GPU.

Hugging Face Hub repo IDs are not fetched: this engine has no network path, so
a repo ID raises ValueError naming the missing local directory.
"""
from __future__ import annotations

import hashlib
import json
import shutil
from pathlib import Path
from typing import Optional

from . import container, decoder, encoder, hub_index

CONFIG_SUFFIXES = {".json", ".txt", ".model", ".tiktoken", ".jinja"}


def _is_repo_id(s: str) -> bool:
    """'user/name' that is not a local path (hub.py:28-43)."""
    if Path(s).exists():
        return False
    if Path(s).suffix in {".safetensors", ".bs", ".json", ".bin"}:
        return False
    parts = s.split("/")
    return len(parts) == 2 and all(parts) and not s.startswith((".", "/", "~"))


def _local_dir(source) -> Path:
    s = str(source)
    if _is_repo_id(s):
        raise ValueError(f"{s!r} looks like a Hub repo ID; this engine reads local directories only "
                         f"(download the model first and pass its directory)")
    p = Path(source)
    if not p.exists():
        raise FileNotFoundError(f"Path not found: {p}")
    return p


def find_safetensors_shards(directory: Path) -> list[Path]:
    """Shards named by model.safetensors.index.json, else model.safetensors, else *.safetensors (hub.py:73-89)."""
    idx = directory / "model.safetensors.index.json"
    if idx.exists():
        data = json.loads(idx.read_text(encoding="utf-8"))
        return [directory / s for s in sorted(set(data["weight_map"].values()))]
    single = directory / "model.safetensors"
    if single.exists():
        return [single]
    return sorted(directory.glob("*.safetensors"))


def shard_output_name(shard_idx: int, total: int) -> str:
    """model.bs, or model-00001-of-0000N.bs (hub.py:92-101)."""
    return "model.bs" if total == 1 else f"model-{shard_idx:05d}-of-{total:05d}.bs"


def scan_cross_shard_duplicates(shards: list[Path]) -> dict[str, dict]:
    """{alias: {"master": name}} for tensors of >= 1024 bytes equal (shape, dtype,
    md5) to an earlier one, in shard then tensor order (hub.py:106-142)."""
    import torch
    from safetensors import safe_open
    seen: dict[tuple, str] = {}
    dups: dict[str, dict] = {}
    for shard in shards:
        with safe_open(str(shard), framework="pt") as f:
            for name in f.keys():
                t = f.get_tensor(name).contiguous()
                raw = t.view(torch.uint8).numpy().tobytes() if t.numel() else b""
                if len(raw) < encoder.TIE_MIN_BYTES:
                    continue
                key = (tuple(t.shape), str(t.dtype).replace("torch.", ""), hashlib.md5(raw).hexdigest())
                if key in seen:
                    dups[name] = {"master": seen[key]}
                else:
                    seen[key] = name
    return dups


def compress_for_hub(source, output_dir, mode: str = "balanced", workers: Optional[int] = None,
                     include_configs: bool = True, overwrite: bool = False,
                     dedupe_cross_shard: bool = True) -> str:
    """Compress a local model directory into .bs shards plus the index (hub.py:145-240)."""
    src = _local_dir(source)
    if src.is_file():
        raise ValueError(f"compress_for_hub expects a model directory, got the file {src}")
    out = Path(output_dir)
    if overwrite and out.exists():
        shutil.rmtree(out)
    out.mkdir(parents=True, exist_ok=True)
    shards = find_safetensors_shards(src)
    if not shards:
        raise FileNotFoundError(f"No *.safetensors files found under {src}")
    dups = scan_cross_shard_duplicates(shards) if dedupe_cross_shard else {}
    bs_paths = []
    for i, shard in enumerate(shards, start=1):
        dst = out / shard_output_name(i, len(shards))
        encoder.compress(shard, dst, mode=mode, exclude_names=set(dups))
        bs_paths.append(dst)
    hub_index.write_index(out, bs_paths, duplicate_map=dups)
    if sum(container.read_header(p)[0]["tensor_count"] for p in bs_paths) >= hub_index.BINARY_INDEX_MIN_TENSORS:
        hub_index.write_binary_index(out, bs_paths)
    if include_configs:
        for p in src.iterdir():
            if p.is_file() and p.suffix in CONFIG_SUFFIXES and p.name != "model.safetensors.index.json":
                shutil.copy2(p, out / p.name)
    return str(out.resolve())


def from_pretrained(repo_or_path, device: str = "cuda", cache_dir: Optional[str] = None,
                    show_progress: bool = False, progress: Optional[bool] = None) -> dict:
    """State dict of a .bs file or a multi-shard directory (hub.py:495-588).
    Every shard is decoded on the GPU (one batched launch per layer group,
    host-to-device copies overlapped with decoding); cross-shard aliases
    share their master's tensor."""
    local = _local_dir(repo_or_path)
    if local.is_file():
        return decoder.load(local, device=device, progress=False)
    index_path = local / hub_index.INDEX_FILENAME
    dup_map: dict = {}
    if index_path.exists():
        index = hub_index.read_index(local)
        shards = hub_index.shard_paths_from_index(local, index)
        dup_map = index["metadata"].get("duplicate_map") or {}
    else:
        shards = sorted(local.glob("*.bs"))
        if not shards:
            raise FileNotFoundError(f"No {hub_index.INDEX_FILENAME} and no .bs files in {local}")
    state: dict = {}
    for shard in shards:
        part = decoder.load(shard, device=device, progress=False)
        clash = set(part) & set(state)
        if clash:
            raise ValueError(f"Duplicate tensor names across shards: {sorted(clash)[:5]}")
        state.update(part)
    for alias, entry in dup_map.items():
        master = entry.get("master") if isinstance(entry, dict) else None
        if master in state and alias not in state:
            state[alias] = state[master]
    return state
