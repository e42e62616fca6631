"""Containers that compress() writes with gpu_optimised / prefer_speed hold
only codecs the reference decodes, routed as the reference routes them
(bigsmall/encoder.py:140-189, tensor_analysis.py:111-119), on the CPU.

The zstd frames are decoded here with the system libzstd's ZSTD_decompress,
independently of this engine's GPU decoder, and the lowcard blob is taken
apart field by field as the reference's special.decode_lowcard reads it
(bigsmall/codecs/special.py:67-85). The selection rules are pinned at their
boundaries with registered codecs of known sizes.
"""
from __future__ import annotations

import ctypes
import ctypes.util
import struct

import numpy as np
import pytest
import torch

from bigsmall_amd import codec_registry, container
from bigsmall_amd.codecs import zstd_host
from bigsmall_amd.encoder import compress

pytestmark = pytest.mark.skipif(not zstd_host.available(), reason="needs the system libzstd")

REFERENCE_CODECS = {"bf16_parallel_v1", "bf16_se_tans", "bf16_se_single_kernel", "special", "zstd", "raw",
                    "tied_ref"}


def _unzstd(frame: bytes) -> bytes:
    L = ctypes.CDLL(ctypes.util.find_library("zstd"))
    L.ZSTD_getFrameContentSize.restype = ctypes.c_ulonglong
    L.ZSTD_getFrameContentSize.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    L.ZSTD_decompress.restype = ctypes.c_size_t
    L.ZSTD_decompress.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t]
    L.ZSTD_isError.restype = ctypes.c_uint
    src = ctypes.create_string_buffer(frame, len(frame))
    n = L.ZSTD_getFrameContentSize(src, len(frame))
    assert n < (1 << 62), "frame without a content size"
    dst = ctypes.create_string_buffer(max(int(n), 1))
    got = L.ZSTD_decompress(dst, int(n), src, len(frame))
    assert not L.ZSTD_isError(got) and got == n
    return dst.raw[:n]


def _read_lowcard(blob: bytes) -> bytes:
    """special.decode_lowcard's reading of the blob (special.py:67-85)."""
    item_bytes, n_unique = struct.unpack_from("<BB", blob, 0)
    p = 2
    uniq = np.frombuffer(blob[p:p + n_unique * item_bytes], np.uint8).reshape(n_unique, item_bytes)
    p += n_unique * item_bytes
    (idx_len,) = struct.unpack_from("<I", blob, p)
    idx = np.frombuffer(_unzstd(blob[p + 4:p + 4 + idx_len]), np.uint8)
    p += 4 + idx_len
    (n_elem,) = struct.unpack_from("<I", blob, p)
    assert p + 4 == len(blob) and idx.size == n_elem
    return uniq[idx].reshape(-1).tobytes()


@pytest.mark.parametrize("item_bytes,n,k", [(2, 4096, 9), (1, 1000, 3), (4, 700, 16), (2, 300, 1)])
def test_lowcard_blob_follows_the_reference_layout(item_bytes, n, k):
    rng = np.random.default_rng(n)
    vals = rng.choice(np.arange(1, 1 << (8 * min(item_bytes, 2)), dtype=np.uint32), k, replace=False)
    words = vals[rng.integers(0, k, n)].astype({1: np.uint8, 2: "<u2", 4: "<u4"}[item_bytes])
    raw = words.tobytes()
    blob, extras = zstd_host.encode_lowcard(raw, item_bytes)
    assert extras == {"item_bytes": item_bytes, "n_unique": len(np.unique(words))}
    assert _read_lowcard(blob) == raw
    # the distinct values are stored ascending, as np.unique gives them
    got = np.frombuffer(blob[2:2 + extras["n_unique"] * item_bytes], words.dtype)
    assert np.array_equal(got, np.unique(words))


def test_lowcard_test_thresholds():
    def t(vals, reps=64):
        return np.repeat(np.asarray(vals, "<u2"), reps).tobytes()
    assert zstd_host.is_lowcard(t(range(16)), 2)            # 16 distinct values: lowcard
    assert not zstd_host.is_lowcard(t(range(17)), 2)        # 17: not
    assert zstd_host.is_lowcard(np.zeros(128, "<u2").tobytes(), 2)          # 256 bytes: lowcard
    assert not zstd_host.is_lowcard(np.zeros(127, "<u2").tobytes(), 2)      # 254 bytes: not
    assert not zstd_host.is_lowcard(np.zeros(300, "<u8").tobytes(), 8)      # items other than 1/2/4 bytes
    # the first 4096 elements decide early: 17 distinct values there, repeats after
    early = np.concatenate([np.arange(4096) % 17, np.zeros(10000, int)]).astype("<u2").tobytes()
    assert zstd_host.count_unique(early, 2) == 17 and not zstd_host.is_lowcard(early, 2)


def test_generic_zstd_entry():
    raw = np.random.default_rng(1).standard_normal(5000).astype(np.float32).tobytes()
    blob, extras = codec_registry.get_codec("zstd")[0](raw)
    assert extras == {"level": 9, "n_bytes": len(raw)} and _unzstd(blob) == raw


@pytest.fixture
def fakes():
    saved = {k: codec_registry.get_codec(k) for k in ("bf16_se_tans", "bf16_se_single_kernel", "bf16_parallel_v1")}
    yield lambda name, size: codec_registry.register_codec(
        name, lambda raw, **_: (b"f" * size, {"fake": name}), lambda b, e, n: b"")
    for k, v in saved.items():
        codec_registry.register_codec(k, *v)


def test_reference_rules_at_their_boundaries(fakes):
    raw = bytes(2 * 2_000_000)                  # 0.6 % of raw = 24,000 bytes > 4096
    T = 1_000_000
    fakes("bf16_se_tans", T)
    sel = lambda **kw: codec_registry.auto_select_reference_codec(raw, "bf16", **kw)[1]
    assert sel() == "bf16_se_tans"                                          # no rule: the stand-in
    fakes("bf16_se_single_kernel", T + 24_000)
    assert sel(prefer_speed=True) == "bf16_se_single_kernel"                # at the tolerance: taken
    fakes("bf16_se_single_kernel", T + 24_001)
    assert sel(prefer_speed=True) == "bf16_se_tans"                         # one byte over: not
    fakes("bf16_parallel_v1", int(T * 1.01))
    assert sel(enable_gpu_parallel=True) == "bf16_parallel_v1"
    fakes("bf16_parallel_v1", int(T * 1.01) + 1)
    assert sel(enable_gpu_parallel=True) == "bf16_se_tans"
    # both flags: the GPU rule is measured against the speed rule's choice
    fakes("bf16_se_single_kernel", T + 20_000)
    fakes("bf16_parallel_v1", int((T + 20_000) * 1.01))
    assert sel(prefer_speed=True, enable_gpu_parallel=True) == "bf16_parallel_v1"
    fakes("bf16_parallel_v1", int((T + 20_000) * 1.01) + 1)
    assert sel(prefer_speed=True, enable_gpu_parallel=True) == "bf16_se_single_kernel"
    # small tensors: the 4096-byte floor of the speed rule
    small = bytes(2 * 10_000)
    fakes("bf16_se_tans", 5000)
    fakes("bf16_se_single_kernel", 5000 + 4096)
    assert codec_registry.auto_select_reference_codec(small, "bf16", prefer_speed=True)[1] == "bf16_se_single_kernel"
    assert codec_registry.auto_select_reference_codec(raw, "fp32")[1] == "zstd"


@pytest.mark.parametrize("flags", [{"gpu_optimised": True}, {"prefer_speed": True},
                                   {"gpu_optimised": True, "prefer_speed": True}])
def test_compress_writes_only_reference_codecs(tmp_path, flags):
    g = torch.Generator().manual_seed(0)
    sd = {"w": (torch.randn(2048, 2048, generator=g) * 0.02).bfloat16(),
          "norm": (1 + torch.randn(4096, generator=g) * 0.01).bfloat16(),
          "mask": torch.tril(torch.ones(64, 64)).bfloat16(),
          "w_tied": None,
          "f32": torch.randn(1000, generator=g),
          "i64": torch.arange(300, dtype=torch.int64),
          "tiny": torch.ones(8).bfloat16()}
    sd["w_tied"] = sd["w"].clone()
    p = tmp_path / "m.bs"
    compress(sd, p, **flags)
    header, data_off = container.read_header(p)
    by = {t["name"]: t for t in header["tensors"]}
    assert {t["codec"] for t in header["tensors"]} <= REFERENCE_CODECS
    assert by["norm"]["codec"] == "special" and by["norm"]["special"] == "lowcard"
    assert by["norm"]["extra"]["special_kind"] == "lowcard"
    assert by["mask"]["codec"] == "special"
    assert by["w_tied"]["codec"] == "tied_ref" and by["tiny"]["codec"] == "raw"
    assert by["f32"]["codec"] == "zstd" and by["i64"]["codec"] == "zstd"
    want_w = {"bf16_parallel_v1"} if flags.get("gpu_optimised") else {"bf16_se_single_kernel", "bf16_se_tans"}
    assert by["w"]["codec"] in want_w
    raw = p.read_bytes()
    blob = lambda t: raw[data_off + t["offset"]:data_off + t["offset"] + t["compressed_bytes"]]
    src = lambda name: sd[name].view(torch.uint8).numpy().tobytes() if sd[name].dtype != torch.bfloat16 \
        else sd[name].view(torch.int16).numpy().tobytes()
    for name in ("norm", "mask"):
        assert _read_lowcard(blob(by[name])) == src(name)
    for name in ("f32", "i64"):
        assert _unzstd(blob(by[name])) == src(name)
