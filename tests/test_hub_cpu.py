"""Multi-shard models on the CPU side: compress_for_hub writes .bs shards,
bigsmall.index.json (with cross-shard aliases in duplicate_map) and, from 100
tensors on, bigsmall.index.bin; the binary index reads back to the JSON's
weight map and to every shard header's offsets, sizes and codecs. Mirrors the
reference's tests/test_opt_step9.py:52-125 and pins the 30-byte record layout
(hub_index.py:36-75) field by field.
"""
from __future__ import annotations

import json
import struct

import pytest
import torch

from bigsmall_amd import container, hub, hub_index
from bigsmall_amd.streaming import StreamingLoader


def _model(n: int, seed: int = 0) -> dict:
    g = torch.Generator().manual_seed(seed)
    return {f"model.layers.{i}.q.weight": (torch.randn(32, 32, generator=g) * 0.02).bfloat16() for i in range(n)}


def _hub_dir(tmp_path, n: int, two_shards: bool = False):
    from safetensors.torch import save_file
    src = tmp_path / "src"
    src.mkdir()
    sd = _model(n)
    if two_shards:
        names = sorted(sd)
        a, b = {k: sd[k] for k in names[: n // 2]}, {k: sd[k] for k in names[n // 2:]}
        emb = (torch.randn(128, 64, generator=torch.Generator().manual_seed(9)) * 0.02).bfloat16()
        a["model.embed_tokens.weight"] = emb
        b["lm_head.weight"] = emb.clone()            # cross-shard duplicate
        save_file(a, str(src / "model-00001-of-00002.safetensors"))
        save_file(b, str(src / "model-00002-of-00002.safetensors"))
        wm = {k: "model-00001-of-00002.safetensors" for k in a} | {k: "model-00002-of-00002.safetensors" for k in b}
        (src / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
        sd |= a | b
    else:
        save_file(sd, str(src / "model.safetensors"))
    (src / "config.json").write_text('{"model_type": "llama"}')
    out = tmp_path / "bs"
    hub.compress_for_hub(src, out, overwrite=True)
    return src, out, sd


def test_binary_index_roundtrip(tmp_path):
    _, out, _ = _hub_dir(tmp_path, 12)
    idx = hub_index.read_index(out)
    shards = hub_index.shard_paths_from_index(out, idx)
    assert [p.name for p in shards] == ["model.bs"]
    b = hub_index.read_binary_index(hub_index.write_binary_index(out, shards))
    assert b["weight_map"] == idx["weight_map"]
    assert b["metadata"]["tensor_count"] == idx["metadata"]["stored_tensor_count"] == 12
    header, _ = container.read_header(shards[0])
    by = {r["name"]: r for r in b["binary"]}
    for t in header["tensors"]:
        r = by[t["name"]]
        assert (r["blob_offset"], r["compressed_bytes"], r["codec"], r["shard_index"]) == \
            (t["offset"], t["compressed_bytes"], t["codec"], 0)


def test_binary_index_written_only_for_large_models(tmp_path):
    (tmp_path / "a").mkdir()
    (tmp_path / "b").mkdir()
    _, big, _ = _hub_dir(tmp_path / "a", 120)
    _, small, _ = _hub_dir(tmp_path / "b", 10)
    assert (big / hub_index.BINARY_INDEX_FILENAME).exists()
    assert not (small / hub_index.BINARY_INDEX_FILENAME).exists()
    assert hub_index.maybe_read_binary_index(small) is None
    assert (big / "config.json").exists()


def test_binary_index_layout(tmp_path):
    _, out, _ = _hub_dir(tmp_path, 3)
    shards = hub_index.shard_paths_from_index(out)
    raw = hub_index.write_binary_index(out, shards).read_bytes()
    assert raw[:8] == b"BSIX\x01\x00\x00\x00"
    n_shards, n_tensors, sec = struct.unpack_from("<III", raw, 8)
    assert (n_shards, n_tensors) == (1, 3)
    assert raw[20:20 + sec] == struct.pack("<H", 8) + b"model.bs"
    p = 20 + sec
    n_codecs = raw[p]
    p += 1
    codecs = []
    for _ in range(n_codecs):
        codecs.append(raw[p + 1:p + 1 + raw[p]].decode())
        p += 1 + raw[p]
    names_len, = struct.unpack_from("<I", raw, p)
    names = raw[p + 4:p + 4 + names_len]
    p += 4 + names_len
    assert len(raw) - p == 3 * 30
    header, _ = container.read_header(shards[0])
    for k, t in enumerate(header["tensors"]):
        no, nl, si, off, nb, ci = struct.unpack_from("<IHHQQB", raw, p + 30 * k)
        assert raw[p + 30 * k + 25:p + 30 * k + 30] == b"\x00" * 5
        assert names[no:no + nl].decode() == t["name"] and si == 0
        assert (off, nb, codecs[ci]) == (t["offset"], t["compressed_bytes"], t["codec"])


def test_read_binary_index_rejects_bad_magic_and_truncation(tmp_path):
    bad = tmp_path / hub_index.BINARY_INDEX_FILENAME
    bad.write_bytes(b"NOTABS\x00\x00\x00\x00\x00\x00\x00\x00")
    with pytest.raises(ValueError, match="Not a BigSmall binary index"):
        hub_index.read_binary_index(bad)
    _, out, _ = _hub_dir(tmp_path, 5)
    good = hub_index.write_binary_index(out, hub_index.shard_paths_from_index(out)).read_bytes()
    bad.write_bytes(good[:-7])
    with pytest.raises(ValueError):
        hub_index.read_binary_index(bad)


def test_cross_shard_duplicates_and_streaming_index(tmp_path):
    _, out, sd = _hub_dir(tmp_path, 8, two_shards=True)
    idx = hub_index.read_index(out)
    meta = idx["metadata"]
    assert meta["shards"] == ["model-00001-of-00002.bs", "model-00002-of-00002.bs"]
    assert meta["duplicate_map"] == {"lm_head.weight": {"master": "model.embed_tokens.weight"}}
    assert meta["tensor_count"] == meta["stored_tensor_count"] + 1 == len(sd)
    assert idx["weight_map"]["lm_head.weight"] == "model-00001-of-00002.bs"
    stored = set()
    for p in hub_index.shard_paths_from_index(out, idx):
        stored |= {t["name"] for t in container.read_header(p)[0]["tensors"]}
    assert "lm_head.weight" not in stored and len(stored) == len(sd) - 1
    with StreamingLoader(out) as L:
        assert set(L.tensor_names()) == set(sd)


def test_repo_ids_are_rejected_without_network(tmp_path):
    with pytest.raises(ValueError, match="repo ID"):
        hub.from_pretrained("someone/some-model")
    with pytest.raises(FileNotFoundError):
        hub.from_pretrained(tmp_path / "missing")
