"""migrate (bigsmall/migrate.py:1-210) on the GPU: a container written in the
reference's own codecs migrates into this engine's GPU formats where they are
smaller, every tensor loads back bit-exactly, kept entries stay byte for byte,
BSCK blobs start on 16-byte boundaries, and dry_run writes nothing."""
from __future__ import annotations

import hashlib
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _model(seed: int = 0) -> dict:
    g = torch.Generator().manual_seed(seed)
    w = lambda *s: (torch.randn(*s, generator=g) * 0.02).bfloat16()
    emb = w(1000, 64)
    return {
        "model.embed_tokens.weight": emb,
        "model.layers.0.self_attn.q_proj.weight": w(256, 512),
        "model.layers.0.self_attn.k_proj.weight": w(128, 512),
        "model.layers.0.mlp.down_proj.weight": w(512, 384),
        "model.layers.0.input_layernorm.weight": (1 + torch.randn(512, generator=g) * 0.01).bfloat16(),
        "model.layers.0.tiny.bias": w(7),
        "lm_head.weight": emb.clone(),
    }


def _blobs(path):
    from bigsmall_amd import container
    header, off = container.read_header(path)
    data = open(path, "rb").read()[off:]
    return header, {t["name"]: (t, data[t["offset"]:t["offset"] + t["compressed_bytes"]]) for t in header["tensors"]}


def _host(tensors: dict) -> dict:
    return {k: v.view(torch.int16).cpu().numpy().copy() if v.dtype == torch.bfloat16 else v.cpu().numpy().copy()
            for k, v in tensors.items()}


def test_migrate_reference_container_into_gpu_formats(tmp_path):
    from bigsmall_amd import compress, load
    from bigsmall_amd.engine import BSCK_CODECS
    from bigsmall_amd.formats import BS_FORMAT_VERSION_V2
    from bigsmall_amd.migrate import migrate
    src = tmp_path / "ref.bs"
    compress(_model(), src, gpu_optimised=True)        # the reference's codecs only
    original = src.read_bytes()
    h0, b0 = _blobs(src)
    _say("[migrate] before:", {t["name"]: t["codec"] for t in h0["tensors"]})
    assert not any(t["codec"] in BSCK_CODECS for t in h0["tensors"])   # bf16_se_tans at these sizes
    want = _host(load(src, device="cuda", progress=False))
    res = migrate(src)
    _say("[migrate] result:", res)
    h1, b1 = _blobs(src)
    assert (tmp_path / "ref.bs.bak").read_bytes() == original
    assert res["tensors_total"] == len(h0["tensors"]) and not res["dry_run"]
    assert res["tensors_migrated"] >= 3 and res["bytes_after"] < res["bytes_before"]
    assert sum(res["codec_changes"].values()) == res["tensors_migrated"]
    assert res["format_version"] == BS_FORMAT_VERSION_V2 and h1["_format_version"] == BS_FORMAT_VERSION_V2
    assert h1["codec_stats"] == {c: sum(t["codec"] == c for t in h1["tensors"]) for c in {t["codec"] for t in h1["tensors"]}}
    for name, (t1, blob1) in b1.items():
        t0, blob0 = b0[name]
        assert t1["md5"] == t0["md5"] and t1["shape"] == t0["shape"]
        if t0["codec"] in ("tied_ref", "raw", "special"):
            assert t1["codec"] == t0["codec"] and blob1 == blob0, name
        if t1["codec"] != t0["codec"]:
            assert len(blob1) < len(blob0), name
        if t1["codec"] in BSCK_CODECS:
            assert t1["offset"] % 16 == 0, name
    assert any(t["codec"] in BSCK_CODECS for t in h1["tensors"])
    got = _host(load(src, device="cuda", progress=False))
    assert got.keys() == want.keys()
    for k in want:
        assert np.array_equal(got[k], want[k]), k


def test_migrate_dry_run_writes_nothing(tmp_path):
    from bigsmall_amd import compress
    from bigsmall_amd.migrate import migrate
    src = tmp_path / "ref.bs"
    compress(_model(1), src, gpu_optimised=True)
    digest = hashlib.sha256(src.read_bytes()).hexdigest()
    dry = migrate(src, dry_run=True)
    assert dry["dry_run"] and hashlib.sha256(src.read_bytes()).hexdigest() == digest
    assert not (tmp_path / "ref.bs.bak").exists() and not (tmp_path / "ref.bs.tmp").exists()
    assert dry["file_size_after"] == dry["file_size_before"]
    real = migrate(src, backup=False)
    assert not (tmp_path / "ref.bs.bak").exists()
    for k in ("tensors_total", "tensors_migrated", "bytes_before", "bytes_after", "codec_changes", "format_version"):
        assert dry[k] == real[k], k
    again = migrate(src, dry_run=True)                 # a migrated file has nothing left to gain
    assert again["tensors_migrated"] == 0 and again["bytes_after"] == again["bytes_before"]
