"""Property-based checks on the CPU (hypothesis), after the reference's
tests/test_property_based.py: for any array the host encoder accepts, the
oracle's BSCK decoder gives it back byte for byte, in every plane mode, state
width, chunk length and coder (rANS; tANS with its states at the stream head or
in a u32 array), and a tANS blob with head states is at most its 256-byte
tail larger than the same chunks with the state array; auto-selection only names registered codecs and its
blob decodes (oracle) to the input; the binary multi-shard index round-trips
arbitrary names, offsets and codecs.
"""
from __future__ import annotations

import numpy as np
import pytest

hyp = pytest.importorskip("hypothesis")
from hypothesis import HealthCheck, given, settings, strategies as st  # noqa: E402

import oracle  # noqa: E402
from bigsmall_amd import codec_registry, hub_index  # noqa: E402
from bigsmall_amd.codecs import bf16_chunked as bc  # noqa: E402

SETTINGS = dict(max_examples=40, deadline=None, suppress_health_check=[HealthCheck.too_slow])


@pytest.fixture(scope="module", autouse=True)
def _oracle():
    oracle.build()


def _words(kind: str, n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    if kind == "gauss":
        x = (rng.standard_normal(n) * 10.0 ** rng.uniform(-4, 1)).astype(np.float32)
        u = x.view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    if kind == "few":
        vals = rng.integers(0, 65536, rng.integers(1, 40)).astype(np.uint16)
        return vals[rng.integers(0, vals.size, n)]
    if kind == "sparse":
        w = _words("gauss", n, seed + 1)
        w[rng.random(n) < rng.uniform(0.3, 0.95)] = 0
        return w
    return rng.integers(0, 65536, n).astype(np.uint16)


@given(kind=st.sampled_from(["gauss", "few", "sparse", "uniform"]), n=st.integers(1, 20_000),
       seed=st.integers(0, 2**31), lanes=st.sampled_from([64, 128, 256]), steps=st.sampled_from([16, 32, 80]),
       mode=st.sampled_from([-1, 0, 1, 2]), coder=st.sampled_from([0, 1, 2]))
@settings(**SETTINGS)
def test_bsck_encode_then_oracle_decode_is_identity(kind, n, seed, lanes, steps, mode, coder):
    w = _words(kind, n, seed)
    if mode == 0 and np.unique(w).size > 256:
        mode = -1
    blob = bc.encode_array(w, steps=steps, mode=mode, lanes=lanes, coder=coder)
    inf = bc.info(blob)
    assert inf.n == n and inf.lanes == lanes and inf.steps == steps and inf.coder == coder
    assert mode < 0 or inf.plane_mode == mode
    assert oracle.chunk_decode(blob, n) == w.tobytes()
    if coder == 2:
        # 2.5 bytes saved per state; the 256-byte tail after the last chunk can take some back
        legacy = bc.encode_array(w, steps=steps, mode=inf.plane_mode, lanes=lanes, coder=1)
        assert len(blob) <= len(legacy) + 256


@given(n=st.integers(1, 50_000), seed=st.integers(0, 2**31))
@settings(**SETTINGS)
def test_fp8_bytes_roundtrip(n, seed):
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, n).astype(np.uint8) if seed % 2 else \
        np.clip(rng.normal(128, 10, n), 0, 255).astype(np.uint8)
    blob = bc.encode_array(b, steps=32)
    assert oracle.chunk_decode(blob, n, elem_bytes=1) == b.tobytes()


@given(kind=st.sampled_from(["gauss", "few", "sparse"]), n=st.integers(256, 20_000), seed=st.integers(0, 2**31),
       dtype=st.sampled_from(["bfloat16", "float8_e4m3fn", "float32"]))
@settings(**SETTINGS)
def test_auto_select_names_a_registered_codec(kind, n, seed, dtype):
    w = _words(kind, n, seed)
    if dtype == "bfloat16":
        raw, fmt, item = w.tobytes(), "bf16", 2
    elif dtype == "float8_e4m3fn":
        raw, fmt, item = w.astype(np.uint8).tobytes(), "fp8", 1
    else:
        raw, fmt, item = w.astype(np.float32).tobytes(), "fp32", 4
    blob, codec, extras = codec_registry.auto_select_codec(raw, fmt, dtype, "model.layers.0.mlp.up_proj.weight",
                                                           (len(raw) // item,), item)
    assert codec in codec_registry.registered_names() or codec == "raw"
    if codec in (bc.CODEC_BF16, bc.CODEC_FP8):
        assert oracle.chunk_decode(blob, len(raw) // item, elem_bytes=item) == raw
    elif codec == "raw":
        assert blob == raw


@given(names=st.lists(st.text(min_size=1, max_size=40), min_size=1, max_size=30, unique=True),
       seed=st.integers(0, 2**31))
@settings(**SETTINGS)
def test_binary_index_roundtrip_arbitrary_names(tmp_path_factory, names, seed):
    import struct
    rng = np.random.default_rng(seed)
    d = tmp_path_factory.mktemp("bsix")
    # a binary index written from synthetic headers: two shards, random offsets/sizes/codecs
    codecs = ["bf16_chunked_v1", "raw", "tied_ref", "bf16_parallel_v1"]
    recs = [(nm, int(rng.integers(0, 2)), int(rng.integers(0, 2**40)), int(rng.integers(0, 2**33)),
             codecs[int(rng.integers(0, 4))]) for nm in names]
    shards = ["model-00001-of-00002.bs", "model-00002-of-00002.bs"]
    name_tab = b"".join(nm.encode() for nm in names)
    body = bytearray(b"BSIX\x01\x00\x00\x00")
    sec = b"".join(struct.pack("<H", len(s)) + s.encode() for s in shards)
    body += struct.pack("<III", 2, len(recs), len(sec)) + sec + bytes([len(codecs)])
    for c in codecs:
        body += bytes([len(c)]) + c.encode()
    body += struct.pack("<I", len(name_tab)) + name_tab
    pos = 0
    for nm, si, off, nb, c in recs:
        ln = len(nm.encode())
        body += struct.pack("<IHHQQB5x", pos, ln, si, off, nb, codecs.index(c))
        pos += ln
    p = d / hub_index.BINARY_INDEX_FILENAME
    p.write_bytes(bytes(body))
    got = hub_index.read_binary_index(p)
    assert [(r["name"], r["shard_index"], r["blob_offset"], r["compressed_bytes"], r["codec"])
            for r in got["binary"]] == recs
    assert got["weight_map"] == {nm: shards[si] for nm, si, _, _, _ in recs}
