"""Routing before codec selection, pinned against the reference's own
`tensor_analysis.analyze_tensors` (bigsmall/tensor_analysis.py:80-132).

tests/golden/routing_vectors.npz holds tensors built on both sides of each
threshold (16 / 17 distinct values, 255 / 256 bytes, a 4096-element first
sample with few values, ties under another dtype, another shape and below
1024 bytes, a tie whose master is lowcard, row-correlated tensors of 16 and 15
rows, item sizes 1, 2, 4 and 8, the C1 layer's RMSNorm vectors) and the
decisions the reference's module made on them (written by
tests/golden/make_golden.py --routing). This build's restatement must make the
same decisions, and its encoder must turn them into the entries the
reference's encoder writes (encoder.py:381-396, 155-168): tied -> tied_ref,
under 512 bytes -> raw, lowcard -> special (containers for the reference's
readers), wpe_delta -> the generic selection (the reference's fallback when
its blosc2 coder is missing, as here).
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from bigsmall_amd import tensor_analysis

GOLDEN = Path(__file__).resolve().parent / "golden" / "routing_vectors.npz"


def _load():
    z = np.load(GOLDEN)                     # plain arrays and JSON strings: no pickle
    meta = json.loads(str(z["meta"]))
    tensors = [dict(m, raw=z[f"raw{i}"].tobytes()) for i, m in enumerate(meta)]
    return tensors, json.loads(str(z["decisions"])), {int(k): v for k, v in json.loads(str(z["tied_map"])).items()}


def test_decisions_match_the_reference():
    tensors, want, want_map = _load()
    got, got_map = tensor_analysis.analyze_tensors(tensors)
    for t, g, w in zip(tensors, got, want):
        assert g == w, (t["name"], g, w)
    assert got_map == want_map
    # every kind is exercised, on both sides of a threshold
    kinds = {d["kind"] for d in want}
    assert kinds == {"tied", "lowcard", "wpe_delta", "generic"}


def test_decisions_with_precomputed_md5s_match():
    import hashlib
    tensors, want, _ = _load()
    got, _ = tensor_analysis.analyze_tensors(tensors, [hashlib.md5(t["raw"]).hexdigest() for t in tensors])
    assert got == want


def test_planted_mistakes_change_decisions():
    """The fixture tells a threshold moved by one from the right one."""
    tensors, want, _ = _load()
    for attr, value in (("MAX_LOWCARD_UNIQUE", 17), ("LOWCARD_MIN_BYTES", 255), ("TIE_MIN_BYTES", 256),
                        ("WPE_MIN_ROWS", 15)):
        old = getattr(tensor_analysis, attr)
        try:
            setattr(tensor_analysis, attr, value)
            got, _ = tensor_analysis.analyze_tensors(tensors)
        finally:
            setattr(tensor_analysis, attr, old)
        assert got != want, attr


@pytest.mark.parametrize("reference_readable", [True, False])
def test_encoder_routes_as_the_reference_encoder(tmp_path, reference_readable):
    import torch
    from bigsmall_amd import codec_registry, container, encoder, formats
    from bigsmall_amd.codecs import zstd_host
    if reference_readable and not zstd_host.available():
        pytest.skip("needs the system libzstd")
    tensors, want, _ = _load()
    dt = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32, "uint8": torch.uint8,
          "int64": torch.int64}
    src = {}
    for t in tensors:
        a = torch.frombuffer(bytearray(t["raw"]), dtype=torch.uint8) if t["raw"] else torch.zeros(0, dtype=torch.uint8)
        src[t["name"]] = a.view(dt[t["dtype"]]).reshape(t["shape"])
    path = tmp_path / "routing.bs"
    encoder.compress(src, path, gpu_optimised=reference_readable)
    header, _ = container.read_header(path)
    entries = {h["name"]: h for h in header["tensors"]}
    for t, d in zip(tensors, want):
        h = entries[t["name"]]
        if d["kind"] == "tied":
            assert h["codec"] == "tied_ref" and h["extra"]["tied_to"] == tensors[d["tied_to"]]["name"], t["name"]
        elif len(t["raw"]) < encoder.RAW_TINY_THRESHOLD:
            assert h["codec"] == "raw", t["name"]
        elif d["kind"] == "lowcard" and reference_readable:
            assert h["codec"] == "special" and h["special"] == "lowcard", t["name"]
        else:
            # the generic selection (wpe_delta included): the codec the registry's rules pick
            fmt = formats.detect_format_from_dtype(t["dtype"]) if t["dtype"] != "int64" else "raw"
            if reference_readable:
                pick = codec_registry.auto_select_reference_codec(t["raw"], fmt, enable_gpu_parallel=True)[1]
            else:
                pick = codec_registry.auto_select_codec(t["raw"], fmt, t["dtype"])[1]
            assert h["codec"] == pick and h["special"] in (None, "gpu_parallel"), (t["name"], h["codec"], pick)
