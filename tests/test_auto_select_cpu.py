"""codec_registry.auto_select_codec against the reference's rules
(bigsmall/codec_registry.py:210-398), on the CPU.

Mirrors of the reference's own tests (tests/test_b4_auto_select.py:40-178):
smallest wins over the first candidate, a registered codec joins the race, the
function never raises, compress() stamps codec_stats summing to the tensor
count. Each tolerance rule is pinned at its boundary with registered codecs of
known sizes (one byte inside the tolerance is taken, one byte outside is not),
and on the reference's golden inputs the decisions follow from the sizes of
the blobs the reference's own encoders wrote (tests/golden/ref_vectors.npz).
"""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from bigsmall_amd import codec_registry, container
from bigsmall_amd.codecs import bf16_parallel, bf16_tans, single_kernel
from bigsmall_amd.encoder import compress


@pytest.fixture
def candidates():
    old = {k: list(v) for k, v in codec_registry.CODEC_CANDIDATES.items()}
    yield codec_registry.CODEC_CANDIDATES
    codec_registry.CODEC_CANDIDATES.clear()
    codec_registry.CODEC_CANDIDATES.update(old)


def _fake(name: str, size: int):
    codec_registry.register_codec(name, lambda raw, **_: (b"f" * size, {"fake": name}), lambda b, e, n: b"")


def _raw(n=64 * 512, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, generator=g) * 0.02).bfloat16().view(torch.uint8).numpy().tobytes()


def test_never_larger_than_first_candidate():
    raw = _raw()
    base, _ = codec_registry.get_codec(codec_registry.CODEC_CANDIDATES["bf16"][0])[0](raw)
    blob, codec, _ = codec_registry.auto_select_codec(raw, "bf16", "BF16")
    assert len(blob) <= len(base) and codec == "bf16_chunked_v1"


def test_registered_codec_joins_the_race(candidates):
    _fake("test_fake_v1", 1)
    candidates["bf16"] = candidates["bf16"] + ["test_fake_v1"]
    assert codec_registry.auto_select_codec(_raw(), "bf16", "BF16")[1] == "test_fake_v1"


def test_ties_go_to_the_earliest_candidate(candidates):
    _fake("tie_a", 100)
    _fake("tie_b", 100)
    candidates["bf16"] = ["tie_a", "tie_b"]
    assert codec_registry.auto_select_codec(_raw(), "bf16", "BF16")[1] == "tie_a"
    candidates["bf16"] = ["tie_b", "tie_a"]
    assert codec_registry.auto_select_codec(_raw(), "bf16", "BF16")[1] == "tie_b"


def test_never_raises_on_garbage_input():
    blob, codec, extras = codec_registry.auto_select_codec(b"\x00", "bf16", "BF16")
    assert codec == "raw" and blob == b"\x00"


def test_gpu_parallel_tolerance_boundary(candidates):
    raw = _raw()
    par = len(bf16_parallel.encode(raw, n_streams=128)[0])
    for base, tol, want in [(par, 0.0, "bf16_parallel_v1"),        # equal size: taken
                            (par - 1, 0.0, "base"),                # one byte larger than the best: not
                            (-(-par // 1.01) + 1, 0.01, "bf16_parallel_v1"),
                            (int(par / 1.01) - 2, 0.01, "base")]:
        _fake("base", int(base))
        candidates["bf16"] = ["base"]
        got = codec_registry.auto_select_codec(raw, "bf16", "BF16", enable_gpu_parallel=True,
                                               gpu_parallel_tolerance=tol)
        assert got[1] == want, (base, tol, par)
        if want == "bf16_parallel_v1":
            assert got[2] == {"n_streams": 128}


def test_prefer_speed_boundaries(candidates):
    raw = _raw(64 * 4096)                        # 512 KiB: tolerances 4096 B (single kernel) and 2048 B (tANS)
    sk = len(single_kernel.encode(raw)[0])
    tans = len(bf16_tans.encode(raw)[0])
    sk_tol, tans_tol = max(4096, int(len(raw) * 0.006)), max(2048, int(len(raw) * 0.0015))
    cases = [(sk - sk_tol, "bf16_se_single_kernel"), (sk - sk_tol - 1, None)]
    for base, want in cases:
        _fake("base", base)
        candidates["bf16"] = ["base"]
        got = codec_registry.auto_select_codec(raw, "bf16", "BF16", prefer_speed=True)[1]
        if want is None:                         # single kernel out of tolerance: tANS within its own?
            want = "bf16_se_tans" if tans <= base + tans_tol else "base"
        assert got == want, (base, sk, tans)
    for base, want in [(tans - tans_tol, "bf16_se_tans"), (tans - tans_tol - 1, "base")]:
        if sk <= base + sk_tol:
            continue                             # the single kernel would win first
        _fake("base", base)
        candidates["bf16"] = ["base"]
        assert codec_registry.auto_select_codec(raw, "bf16", "BF16", prefer_speed=True)[1] == want
    candidates["bf16"] = ["bf16_se_tans"]          # a tANS candidate disables the speed rule
    assert codec_registry.auto_select_codec(raw, "bf16", "BF16", prefer_speed=True)[1] == "bf16_se_tans"


def test_rans_tie_break_boundary(candidates):
    raw = _raw()
    tol = max(1024, int(len(raw) * 0.0001))
    for ac, rans, want in [(5000, 5000 + tol, "bf16_se_rans"), (5000, 5001 + tol, "bf16_se_ac"),
                           (5000, 4000, "bf16_se_rans")]:
        _fake("bf16_se_ac", ac)
        _fake("bf16_se_rans", rans)
        candidates["bf16"] = ["bf16_se_rans", "bf16_se_ac"]
        assert codec_registry.auto_select_codec(raw, "bf16", "BF16")[1] == want, (ac, rans)
    for name in ("bf16_se_ac", "bf16_se_rans"):
        codec_registry._REGISTRY.pop(name)


def test_golden_inputs_follow_the_reference_blob_sizes(golden, candidates):
    """On each golden input, the selections follow from the sizes of the
    reference encoder's own blobs for it: bf16_parallel_v1 (64 streams) within
    1 % of a bf16_se_tans-only candidate list, and prefer_speed's choice over
    this engine's bf16_chunked_v1."""
    n = 0
    for k in sorted(golden):
        if not (k.startswith("par1_") and k.endswith("_N64")):
            continue
        name = k[len("par1_"):-len("_N64")]
        raw = golden[f"in_{name}"].astype("<u2").tobytes()
        ref_par, ref_tans, ref_sk = len(golden[k]), len(golden[f"tans_{name}"]), len(golden[f"sk_{name}"])
        candidates["bf16"] = ["bf16_se_tans"]
        got = codec_registry.auto_select_codec(raw, "bf16", "BF16", enable_gpu_parallel=True,
                                               gpu_parallel_n_streams=64)
        assert got[1] == ("bf16_parallel_v1" if ref_par <= int(ref_tans * 1.01) else "bf16_se_tans"), name
        assert got[0] == (golden[k].tobytes() if got[1] == "bf16_parallel_v1" else golden[f"tans_{name}"].tobytes())
        candidates["bf16"] = ["bf16_chunked_v1"]
        base = len(codec_registry.get_codec("bf16_chunked_v1")[0](raw)[0])
        want = ("bf16_se_single_kernel" if ref_sk <= base + max(4096, int(len(raw) * 0.006)) else
                "bf16_se_tans" if ref_tans <= base + max(2048, int(len(raw) * 0.0015)) else "bf16_chunked_v1")
        assert codec_registry.auto_select_codec(raw, "bf16", "BF16", prefer_speed=True)[1] == want, name
        n += 1
    assert n >= 6


def test_compress_gpu_optimised_writes_reference_formats(tmp_path):
    """compress(gpu_optimised=True) stores bf16_parallel_v1 when it is within
    1 % of the best candidate (so the reference can read the file), promotes the
    container to version 2, and codec_stats sums to the tensor count
    (tests/test_b4_auto_select.py:140-160)."""
    import oracle
    oracle.build()
    g = torch.Generator().manual_seed(4)
    src = {"model.layers.0.mlp.up_proj.weight": (torch.randn(2048, 2048, generator=g) * 0.02).bfloat16(),
           "model.layers.0.input_layernorm.weight": (1 + torch.randn(256, generator=g) * 0.01).bfloat16(),
           "bias": torch.zeros(8, dtype=torch.bfloat16)}
    for kw, codec in [({"gpu_optimised": True}, "bf16_parallel_v1"), ({"prefer_speed": True}, None)]:
        p = tmp_path / f"m{len(kw)}{codec}.bs"
        compress(src, p, **kw)
        header, off = container.read_header(p)
        stats = header["codec_stats"]
        assert sum(stats.values()) == header["tensor_count"] == 3
        t = next(t for t in header["tensors"] if t["name"].endswith("up_proj.weight"))
        if codec:
            raw = src[t["name"]].view(torch.uint8).numpy().tobytes()
            par, base = len(bf16_parallel.encode(raw)[0]), len(codec_registry.get_codec("bf16_chunked_v1")[0](raw)[0])
            assert par <= base * 1.01                           # a large Gaussian tensor: within the tolerance
            assert t["codec"] == codec and int.from_bytes(p.read_bytes()[4:6], "little") == 2
        else:
            assert t["codec"] in ("bf16_se_single_kernel", "bf16_se_tans", "bf16_chunked_v1")
        blob = container.read_blob(p, header, off, header["tensors"].index(t))
        dec = {"bf16_parallel_v1": oracle.par1_decode, "bf16_se_tans": oracle.tans_decode,
               "bf16_se_single_kernel": oracle.sk_decode, "bf16_chunked_v1": oracle.chunk_decode}[t["codec"]]
        want = src[t["name"]].view(torch.int16).numpy().tobytes()
        assert dec(blob, 2048 * 2048) == want


def _sparse(n, seed=0):
    g = torch.Generator().manual_seed(seed)
    y = (torch.randn(n, generator=g) * 0.02).bfloat16()
    y[torch.randperm(n, generator=g)[: n // 2]] = 0
    return y.view(torch.uint8).numpy().tobytes()


def test_compact_tensors_take_the_table_ans_form(candidates):
    """The engine's compact-tANS rule: with bf16_chunked_tans_v1 after
    bf16_chunked_v1 in the list (the default), a compact-mode rANS winner
    yields to the tANS blob when that is at most compact_tans_tolerance
    larger; a dense winner is kept without encoding tANS; a list without the
    tANS codec forces rANS, one with only it forces tANS."""
    from bigsmall_amd.codecs import bf16_chunked as bc
    raw = _sparse(4_000_000)
    rans = codec_registry.get_codec(bc.CODEC_BF16)[0](raw)[0]
    tans = codec_registry.get_codec(bc.CODEC_BF16_TANS)[0](raw)[0]
    assert bc.info(rans).plane_mode == bc.MODE_COMPACT and len(rans) < len(tans) <= len(rans) * 1.01
    assert candidates["bf16"] == [bc.CODEC_BF16, bc.CODEC_BF16_TANS]
    blob, codec, _ = codec_registry.auto_select_codec(raw, "bf16", "BF16")
    assert codec == bc.CODEC_BF16_TANS and blob == tans
    # the tolerance boundary: half a byte above the size difference admits it, half a byte below does not
    d = len(tans) - len(rans)
    assert codec_registry.auto_select_codec(raw, "bf16", "BF16",
                                            compact_tans_tolerance=(d + 0.5) / len(rans))[1] == bc.CODEC_BF16_TANS
    assert codec_registry.auto_select_codec(raw, "bf16", "BF16",
                                            compact_tans_tolerance=(d - 0.5) / len(rans))[1] == bc.CODEC_BF16
    candidates["bf16"] = [bc.CODEC_BF16]
    assert codec_registry.auto_select_codec(raw, "bf16", "BF16")[1] == bc.CODEC_BF16
    candidates["bf16"] = [bc.CODEC_BF16_TANS]
    assert codec_registry.auto_select_codec(raw, "bf16", "BF16")[1] == bc.CODEC_BF16_TANS


def test_dense_and_small_compact_tensors_keep_rans(candidates, monkeypatch):
    from bigsmall_amd.codecs import bf16_chunked as bc
    calls = []
    enc = codec_registry.get_codec(bc.CODEC_BF16_TANS)
    monkeypatch.setitem(codec_registry._REGISTRY, bc.CODEC_BF16_TANS,
                        (lambda raw, **ctx: calls.append(1) or enc[0](raw, **ctx), enc[1]))
    assert codec_registry.auto_select_codec(_raw(2_000_000), "bf16", "BF16")[1] == bc.CODEC_BF16
    assert not calls                         # a dense winner: the tANS form is not encoded
    # a small compact tensor: the stored 16 KB decode table puts tANS more than 1 % above
    assert codec_registry.auto_select_codec(_sparse(300_000), "bf16", "BF16")[1] == bc.CODEC_BF16
    assert calls
