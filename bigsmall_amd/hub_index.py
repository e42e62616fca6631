"""Multi-shard index: `bigsmall.index.json` and its binary form
`bigsmall.index.bin` (the reference's formats, bigsmall/hub_index.py:79-402),
so a model split over several .bs shards loads as one unit.

JSON index:
    {"metadata": {bigsmall_version, container_version, format_version, format,
                  mode, model_type, total_size, total_raw_size, ratio_pct,
                  shard_count, tensor_count, stored_tensor_count, shards,
                  [duplicate_map]},
     "weight_map": {tensor_name: shard_filename}}
`duplicate_map` ({alias: {"master": name}}) lists cross-shard tied tensors that
are stored once; aliases appear in the weight map under the master's shard.

Binary index (little-endian):
    "BSIX" | u8 version = 1 | 3 zero bytes | u32 n_shards | u32 n_tensors
    u32 shard-name section size | per shard: u16 length, UTF-8 name
    u8 n_codecs | per codec: u8 length, UTF-8 name
    u32 name-table size | UTF-8 tensor names (each distinct name once)
    per tensor, 30 bytes: u32 name offset, u16 name length, u16 shard index,
        u64 blob offset, u64 compressed bytes, u8 codec index, 5 zero bytes
The byte layouts are kept identical to the reference's so either side reads
the other's files.
"""
from __future__ import annotations

import json
import struct
from pathlib import Path
from typing import Any, Optional

from . import container

INDEX_FILENAME = "bigsmall.index.json"
BINARY_INDEX_FILENAME = "bigsmall.index.bin"
BINARY_INDEX_MIN_TENSORS = 100
BINARY_INDEX_MAGIC = b"BSIX"
BINARY_INDEX_VERSION = 1
_RECORD = struct.Struct("<IHHQQB5x")
assert _RECORD.size == 30


def _container_version(path: Path) -> int:
    with open(path, "rb") as f:
        head = f.read(6)
    if len(head) < 6 or head[:4] != container.MAGIC:
        raise ValueError(f"{path}: not a BigSmall container")
    return struct.unpack_from("<H", head, 4)[0]


def build_index(shard_paths, model_type: Optional[str] = None,
                duplicate_map: Optional[dict] = None) -> dict[str, Any]:
    """Index dict for the given shards, in order (hub_index.py:79-171). A tensor
    in two shards, or shards of different container versions, raise ValueError."""
    shards = [Path(p) for p in shard_paths]
    if not shards:
        raise ValueError("build_index needs at least one shard")
    weight_map: dict[str, str] = {}
    total_size = total_raw = stored = 0
    fmts, modes, types, versions = set(), set(), set(), set()
    for shard in shards:
        inf = container.info(shard)
        total_size += int(inf["file_size"])
        total_raw += int(inf["estimated_raw_bytes"])
        stored += int(inf["tensor_count"])
        fmts.add(inf["format"])
        modes.add(inf["mode"])
        types.add(inf["model_type"])
        versions.add(_container_version(shard))
        header, _ = container.read_header(shard)
        for t in header["tensors"]:
            prev = weight_map.get(t["name"])
            if prev is not None and prev != shard.name:
                raise ValueError(f"Tensor {t['name']!r} appears in two shards: {prev} and {shard.name}")
            weight_map[t["name"]] = shard.name
    if len(versions) != 1:
        raise ValueError(f"Mixed container versions across shards: {sorted(versions)}")
    dup = dict(duplicate_map or {})
    for alias, entry in dup.items():
        master = entry.get("master") if isinstance(entry, dict) else None
        if master in weight_map and alias not in weight_map:
            weight_map[alias] = weight_map[master]
    from . import __version__
    version = next(iter(versions))
    metadata = {
        "bigsmall_version": str(__version__),
        "container_version": version,
        "format_version": version,
        "format": next(iter(fmts)) if len(fmts) == 1 else "mixed",
        "mode": next(iter(modes)) if len(modes) == 1 else "mixed",
        "model_type": model_type or (next(iter(types)) if len(types) == 1 else "llm"),
        "total_size": total_size,
        "total_raw_size": total_raw,
        "ratio_pct": (total_size / total_raw * 100.0) if total_raw else 0.0,
        "shard_count": len(shards),
        "tensor_count": stored + len(dup),
        "stored_tensor_count": stored,
        "shards": [p.name for p in shards],
    }
    if dup:
        metadata["duplicate_map"] = dup
    return {"metadata": metadata, "weight_map": weight_map}


def write_index(directory, shard_paths, model_type: Optional[str] = None,
                duplicate_map: Optional[dict] = None) -> Path:
    out = Path(directory) / INDEX_FILENAME
    out.write_text(json.dumps(build_index(shard_paths, model_type, duplicate_map), indent=2), encoding="utf-8")
    return out


def read_index(directory_or_path) -> dict[str, Any]:
    p = Path(directory_or_path)
    if p.is_dir():
        p = p / INDEX_FILENAME
    if not p.exists():
        raise FileNotFoundError(f"No {INDEX_FILENAME} at {p}")
    return json.loads(p.read_text(encoding="utf-8"))


def shard_paths_from_index(directory, index: Optional[dict] = None) -> list[Path]:
    directory = Path(directory)
    index = index if index is not None else read_index(directory)
    return [directory / name for name in index["metadata"]["shards"]]


def write_binary_index(directory, shard_paths) -> Path:
    """bigsmall.index.bin for the given shards (hub_index.py:228-303)."""
    shards = [Path(p) for p in shard_paths]
    records = []
    for si, shard in enumerate(shards):
        header, _ = container.read_header(shard)
        for t in header["tensors"]:
            records.append((t["name"], si, int(t.get("offset", 0)), int(t.get("compressed_bytes", 0)),
                            t.get("codec") or "?"))
    names = bytearray()
    name_at: dict[str, tuple[int, int]] = {}
    codecs: dict[str, int] = {}
    for name, _, _, _, codec in records:
        if name not in name_at:
            b = name.encode("utf-8")
            name_at[name] = (len(names), len(b))
            names += b
        codecs.setdefault(codec, len(codecs))
    if len(codecs) > 255:
        raise ValueError(f"binary index: {len(codecs)} distinct codec names (at most 255)")
    shard_sec = bytearray()
    for shard in shards:
        b = shard.name.encode("utf-8")
        if len(b) > 0xFFFF:
            raise ValueError(f"shard name too long for the binary index: {shard.name!r}")
        shard_sec += struct.pack("<H", len(b)) + b
    out = bytearray(BINARY_INDEX_MAGIC + bytes([BINARY_INDEX_VERSION, 0, 0, 0]))
    out += struct.pack("<III", len(shards), len(records), len(shard_sec)) + shard_sec
    out += bytes([len(codecs)])
    for codec in codecs:
        b = codec.encode("utf-8")
        if len(b) > 255:
            raise ValueError(f"codec name too long: {codec!r}")
        out += bytes([len(b)]) + b
    out += struct.pack("<I", len(names)) + names
    for name, si, off, nbytes, codec in records:
        o, ln = name_at[name]
        out += _RECORD.pack(o, ln, si, off, nbytes, codecs[codec])
    path = Path(directory) / BINARY_INDEX_FILENAME
    path.write_bytes(bytes(out))
    return path


def read_binary_index(path) -> dict[str, Any]:
    """Parse bigsmall.index.bin (hub_index.py:306-391): metadata, weight_map
    and the per-tensor records (shard, blob offset, compressed bytes, codec)."""
    p = Path(path)
    if p.is_dir():
        p = p / BINARY_INDEX_FILENAME
    if not p.exists():
        raise FileNotFoundError(f"No binary index at {p}")
    b = p.read_bytes()
    pos = 0

    def take(n: int) -> bytes:
        nonlocal pos
        if pos + n > len(b):
            raise ValueError(f"binary index truncated at byte {pos}")
        s = b[pos:pos + n]
        pos += n
        return s

    if take(4) != BINARY_INDEX_MAGIC:
        raise ValueError(f"Not a BigSmall binary index: {p}")
    version = take(4)[0]
    if version != BINARY_INDEX_VERSION:
        raise ValueError(f"Unsupported binary index version {version} (expected {BINARY_INDEX_VERSION})")
    n_shards, n_tensors, sec = struct.unpack("<III", take(12))
    shard_sec = take(sec)
    shards, q = [], 0
    for _ in range(n_shards):
        ln, = struct.unpack_from("<H", shard_sec, q)
        shards.append(shard_sec[q + 2:q + 2 + ln].decode("utf-8"))
        q += 2 + ln
    codecs = []
    for _ in range(take(1)[0]):
        codecs.append(take(take(1)[0]).decode("utf-8"))
    name_size, = struct.unpack("<I", take(4))
    names = take(name_size)
    records, weight_map = [], {}
    for _ in range(n_tensors):
        no, nl, si, off, nbytes, ci = _RECORD.unpack(take(_RECORD.size))
        if si >= n_shards or ci >= len(codecs) or no + nl > len(names):
            raise ValueError("binary index record out of range")
        name = names[no:no + nl].decode("utf-8")
        records.append({"name": name, "shard_index": si, "shard": shards[si], "blob_offset": off,
                        "compressed_bytes": nbytes, "codec": codecs[ci]})
        weight_map[name] = shards[si]
    return {"metadata": {"shards": shards, "shard_count": n_shards, "tensor_count": n_tensors,
                         "binary_index_version": version},
            "weight_map": weight_map, "binary": records}


def maybe_read_binary_index(directory) -> Optional[dict[str, Any]]:
    p = Path(directory) / BINARY_INDEX_FILENAME
    if not p.exists():
        return None
    try:
        return read_binary_index(p)
    except (ValueError, FileNotFoundError):
        return None
