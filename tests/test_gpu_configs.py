"""GPU parity at the benchmark configurations (bit-exact, md5 per tensor).

C0  4096x4096 bf16 N(0, 0.02): this engine's encoder with auto-selection, and
    the reference's formats (oracle encoders, byte-identical to the reference's).
C2  the full Llama-3-8B-shaped model (32 layers, untied 128256x4096
    embed_tokens and lm_head, about 16 GB of bf16) written to a .bs file and
    read back into HBM by decoder.load's pinned host-to-device layer pipeline,
    all 290 tensors compared bit-exact; and two layers at their real shapes
    from the CPU generator.
C3  8192x8192 stress: (a) Student-t df=3 at std 0.02, (b) half exact zeros,
    (c) fp8 e4m3 of N(0, 1) plus its bf16 residual; "forced rANS" = the
    reference's bf16_parallel_v1 and this engine's bf16_chunked_v1 /
    fp8_chunked_v1, "forced tANS" = this engine's bf16_chunked_tans_v1 /
    fp8_chunked_tans_v1 (table ANS) and the reference's bf16_se_tans (its Numba
    rANS codec), forced through a CODEC_CANDIDATES override.
C4  KV cache blocks of 256 tokens, K and V [8 heads, 32768 tokens, 128] per layer
    scaled per head by U[0.5, 2], 64 random blocks per layer decoded in one launch:
    all 32 layers encoded on the GPU from device K/V and all 4,096 decoded blocks
    compared; and two layers through the host encoder.
"""
from __future__ import annotations

import hashlib
import struct
import sys

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _words(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)


def _gpu_words(t) -> bytes:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).tobytes()


@pytest.fixture(scope="module", autouse=True)
def _setup():
    assert torch.cuda.is_available()
    oracle.build()


def _check_ref(codec, blob, words):
    from bigsmall_amd.codecs import _refstreams
    got = _refstreams.decode_host(codec, blob, words.size)
    assert hashlib.md5(got).hexdigest() == hashlib.md5(words.tobytes()).hexdigest(), codec


def _check_bsck(words, **kw):
    from bigsmall_amd.codecs import bf16_chunked as bc
    blob = bc.encode_array(words, **kw)
    eb = words.dtype.itemsize
    got = bc.decode(blob, {}, words.size, elem_bytes=eb)
    assert hashlib.md5(got).hexdigest() == hashlib.md5(words.tobytes()).hexdigest(), kw
    return len(blob) / words.nbytes


def test_c0_4096_square(tmp_path):
    from bigsmall_amd.decoder import load
    from bigsmall_amd.encoder import compress
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(4096, 4096, generator=g) * 0.02).bfloat16()
    p = tmp_path / "c0.bs"
    compress({"w": w}, p)
    _say("[c0] engine container")
    assert torch.equal(load(p)["w"].cpu().view(torch.int16), w.view(torch.int16))
    words = _words(w)
    for codec, enc in [("bf16_parallel_v1", oracle.par1_encode), ("bf16_se_tans", oracle.tans_encode),
                       ("bf16_se_single_kernel", oracle.sk_encode)]:
        _say(f"[c0] {codec}")
        _check_ref(codec, enc(words), words)


def _stress(kind: str) -> np.ndarray:
    g = torch.Generator().manual_seed(3)
    n = 8192 * 8192
    if kind == "studentt":
        # Student-t, 3 degrees of freedom, from the seeded generator: Z / sqrt(chi2_3 / 3)
        z = torch.randn(n, generator=g)
        chi2 = sum(torch.randn(n, generator=g) ** 2 for _ in range(3))
        x = z / torch.sqrt(chi2 / 3.0) * (0.02 / np.sqrt(3.0))
    else:
        x = torch.randn(n, generator=g) * 0.02
    w = _words(x.bfloat16())
    if kind == "halfzero":
        w = w.copy()
        w[torch.randperm(n, generator=g).numpy()[: n // 2]] = 0
    return w


@pytest.mark.parametrize("kind", ["studentt", "halfzero"])
def test_c3_bf16_stress_forced_rans(kind):
    w = _stress(kind)
    for mode in (-1, 1, 2):
        _say(f"[c3] {kind} bf16_chunked_v1 mode={mode}")
        _check_bsck(w, mode=mode)
    _say(f"[c3] {kind} bf16_parallel_v1")
    _check_ref("bf16_parallel_v1", oracle.par1_encode(w), w)


def _forced(fmt: str, codec: str, words):
    """Encode through codec_registry.auto_select_codec with CODEC_CANDIDATES
    overridden to one codec (the reference's forcing mechanism,
    tests/test_b4_auto_select.py:121-132 there), decode through the decoder's
    dispatch, compare md5."""
    from bigsmall_amd import codec_registry, decoder
    saved = dict(codec_registry.CODEC_CANDIDATES)
    try:
        codec_registry.CODEC_CANDIDATES[fmt] = [codec]
        raw = words.tobytes()
        blob, name, extras = codec_registry.auto_select_codec(raw, fmt, "float8_e4m3fn" if fmt == "fp8" else "bfloat16")
    finally:
        codec_registry.CODEC_CANDIDATES.clear()
        codec_registry.CODEC_CANDIDATES.update(saved)
    assert name == codec
    t = {"name": "c3", "codec": name, "extra": extras, "shape": [words.size],
         "dtype": "float8_e4m3fn" if fmt == "fp8" else "bfloat16"}
    got = decoder._decode_blob(t, blob)
    assert hashlib.md5(got).hexdigest() == hashlib.md5(raw).hexdigest(), codec
    assert got == oracle.chunk_decode(blob, words.size, words.dtype.itemsize), codec
    return blob


@pytest.mark.parametrize("kind", ["studentt", "halfzero"])
def test_c3_bf16_stress_forced_tans(kind):
    w = _stress(kind)
    _say(f"[c3] {kind} bf16_chunked_tans_v1 (forced tANS, this engine's format)")
    blob = _forced("bf16", "bf16_chunked_tans_v1", w)
    assert blob[28] == 2 and blob[6] == (2 if kind == "halfzero" else 1)
    assert struct.unpack_from("<IH", blob, 16) == (224, 256)     # the tANS codec's chunk geometry
    for mode in (1, 2):
        _say(f"[c3] {kind} bf16_chunked_tans_v1 mode={mode}")
        _check_bsck(w, mode=mode, coder=2, lanes=256, steps=64)
    # the earlier tANS layout (u32 initial states, 128 lanes) still decodes at full size
    _say(f"[c3] {kind} tANS coder 1 (u32 state array)")
    _check_bsck(w, coder=1, lanes=128, steps=128)
    _say(f"[c3] {kind} bf16_se_tans (the reference's forced-tANS format)")
    _check_ref("bf16_se_tans", oracle.tans_encode(w), w)


def test_c3_fp8_and_residual():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(8192 * 8192, generator=g)
    f8 = x.to(torch.float8_e4m3fn)
    resid = (x - f8.float()).bfloat16()
    b8 = f8.view(torch.uint8).numpy()
    for coder, codec in ((0, "fp8_chunked_v1"), (2, "fp8_chunked_tans_v1")):
        _say(f"[c3] fp8 e4m3 {codec} (exponent pairs, then byte symbols)")
        blob = _forced("fp8", codec, b8)
        assert blob[6] == 3 and blob[28] == coder
        _check_bsck(b8, mode=0, coder=coder)
    rw = _words(resid)
    _say("[c3] residual bf16_chunked_v1 / bf16_parallel_v1 (forced rANS)")
    _forced("bf16", "bf16_chunked_v1", rw)
    _check_ref("bf16_parallel_v1", oracle.par1_encode(rw), rw)
    _say("[c3] residual bf16_chunked_tans_v1 / bf16_se_tans (forced tANS)")
    assert _forced("bf16", "bf16_chunked_tans_v1", rw)[28] == 2
    _check_ref("bf16_se_tans", oracle.tans_encode(rw), rw)


def test_c4_kv_blocks():
    from bigsmall_amd.kv_cache_manager import CompressedKVCache
    g = torch.Generator().manual_seed(5)
    cache = CompressedKVCache(device="cuda")
    src = {}
    for layer in range(2):
        s = torch.empty(8, 1, 1).uniform_(0.5, 2.0, generator=g)
        k = (torch.randn(8, 32768, 128, generator=g) * s).bfloat16()
        v = (torch.randn(8, 32768, 128, generator=g) * s).bfloat16()
        assert cache.set_blocks(layer, k, v, block_tokens=256) == 128
        src[layer] = (k, v)
    rng = np.random.default_rng(6)
    req = [(layer, rng.choice(128, 64, replace=False)) for layer in range(2)]
    _say("[c4] 2 layers x 64 blocks x (K, V) in one launch")
    out = cache.get_blocks_multi(req)
    for (layer, ids), (kb, vb) in zip(req, out):
        k, v = src[layer]
        for j, b in enumerate(ids):
            assert _gpu_words(kb[j]) == _words(k[:, b * 256:(b + 1) * 256]).tobytes()
            assert _gpu_words(vb[j]) == _words(v[:, b * 256:(b + 1) * 256]).tobytes()
    assert 0.6 < cache.compression_ratio() < 0.85


def test_c2_layers_at_real_shape(tmp_path):
    from bigsmall_amd.decoder import load
    from bigsmall_amd.encoder import compress
    g = torch.Generator().manual_seed(7)
    shapes = {"self_attn.q_proj": (4096, 4096), "self_attn.k_proj": (1024, 4096), "self_attn.v_proj": (1024, 4096),
              "self_attn.o_proj": (4096, 4096), "mlp.gate_proj": (14336, 4096), "mlp.up_proj": (14336, 4096),
              "mlp.down_proj": (4096, 14336)}
    t = {"model.embed_tokens.weight": (torch.randn(8192, 4096, generator=g) * 0.02).bfloat16()}
    for i in range(2):
        for k, s in shapes.items():
            t[f"model.layers.{i}.{k}.weight"] = (torch.randn(*s, generator=g) * 0.02).bfloat16()
        for k in ("input_layernorm", "post_attention_layernorm"):
            t[f"model.layers.{i}.{k}.weight"] = (1 + torch.randn(4096, generator=g) * 0.01).bfloat16()
    p = tmp_path / "c2.bs"
    compress(t, p)
    _say("[c2] load 2 layers + embedding slice")
    out = load(p)
    for k, v in t.items():
        assert torch.equal(out[k].cpu().view(torch.int16), v.view(torch.int16)), k


@pytest.mark.timeout(900)
def test_c2_full_model_load(tmp_path):
    """C2 at full size: 32 Llama-3-8B-shaped layers (seeded N(0, 0.02)
    matrices, 1 + N(0, 0.01) norms) and untied 128256x4096 embed_tokens /
    lm_head: 8,030,257,152 weights, drawn on the GPU from a seeded generator.
    compress() writes the .bs file; decoder.load decodes it into HBM through
    the pinned host-to-device pipeline (bigsmall/decoder.py:100-157, 301-310);
    every one of the 290 tensors is compared with its source on the device."""
    import time
    from bigsmall_amd import container
    from bigsmall_amd.decoder import load
    from bigsmall_amd.encoder import compress
    t0 = time.time()
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(8)
    shapes = {"self_attn.q_proj": (4096, 4096), "self_attn.k_proj": (1024, 4096), "self_attn.v_proj": (1024, 4096),
              "self_attn.o_proj": (4096, 4096), "mlp.gate_proj": (14336, 4096), "mlp.up_proj": (14336, 4096),
              "mlp.down_proj": (4096, 14336)}
    rnd = lambda *s: (torch.randn(*s, generator=g, device=dev) * 0.02).bfloat16()
    src = {"model.embed_tokens.weight": rnd(128256, 4096)}
    for i in range(32):
        for k, s in shapes.items():
            src[f"model.layers.{i}.{k}.weight"] = rnd(*s)
        for k in ("input_layernorm", "post_attention_layernorm"):
            src[f"model.layers.{i}.{k}.weight"] = (1 + torch.randn(4096, generator=g, device=dev) * 0.01).bfloat16()
    src["lm_head.weight"] = rnd(128256, 4096)
    n = sum(v.numel() for v in src.values())
    assert len(src) == 290 and n == 8_030_257_152
    torch.cuda.synchronize()
    _say(f"[c2] full model drawn: {len(src)} tensors, {n} weights ({time.time() - t0:.0f}s)")
    p = tmp_path / "llama3_8b_shape.bs"
    compress(src, p)
    header, _ = container.read_header(p)
    assert len(header["tensors"]) == 290 and all(t["codec"] == "bf16_chunked_v1" for t in header["tensors"]
                                                 if "norm" not in t["name"])
    _say(f"[c2] written {p.stat().st_size / 1e9:.2f} GB ({time.time() - t0:.0f}s)")
    out = load(p, device="cuda")
    torch.cuda.synchronize()
    _say(f"[c2] decoder.load done ({time.time() - t0:.0f}s)")
    assert list(out) == list(src)
    for k, v in src.items():
        o = out[k]
        assert o.device == dev and o.dtype == v.dtype and tuple(o.shape) == tuple(v.shape), k
        assert torch.equal(o.view(torch.int16), v.view(torch.int16)), k
    _say(f"[c2] all 290 tensors bit-exact ({time.time() - t0:.0f}s)")


@pytest.mark.timeout(600)
def test_c4_all_layers_all_blocks():
    """C4 at full size: K and V [8, 32768, 128] for each of 32 layers, N(0, 1)
    scaled per (layer, head) by U[0.5, 2], drawn on the GPU from a seeded
    generator and encoded there by set_blocks in 256-token blocks
    (bigsmall/kv_cache_manager.py:39-56 keys one blob per layer; blocks are
    this engine's addition); 64 seeded random blocks per layer for K and V,
    4,096 blocks, decoded by one get_blocks_multi launch and each compared
    with its source block."""
    from bigsmall_amd.kv_cache_manager import CompressedKVCache
    dev = torch.device("cuda", 0)
    gs = torch.Generator().manual_seed(9)
    gd = torch.Generator(device=dev).manual_seed(10)
    cache = CompressedKVCache(device="cuda")
    kv = []
    for layer in range(32):
        s = torch.empty(8, 1, 1).uniform_(0.5, 2.0, generator=gs).to(dev)
        k = (torch.randn(8, 32768, 128, generator=gd, device=dev) * s).bfloat16()
        v = (torch.randn(8, 32768, 128, generator=gd, device=dev) * s).bfloat16()
        assert cache.set_blocks(layer, k, v, block_tokens=256) == 128
        kv.append((k, v))
    _say("[c4] 32 layers encoded on the GPU")
    rng = np.random.default_rng(11)
    req = [(layer, rng.choice(128, 64, replace=False)) for layer in range(32)]
    out = cache.get_blocks_multi(req)
    _say("[c4] 32 x 64 x (K, V) blocks decoded in one launch")
    checked = 0
    for (layer, ids), (kb, vb) in zip(req, out):
        idx = torch.as_tensor(ids, dtype=torch.long, device=dev)
        for got, full in ((kb, kv[layer][0]), (vb, kv[layer][1])):
            want = full.view(8, 128, 256, 128).index_select(1, idx).movedim(1, 0)
            assert got.shape == want.shape
            for j in range(len(ids)):
                assert torch.equal(got[j].view(torch.int16), want[j].view(torch.int16)), (layer, j)
                checked += 1
    assert checked == 4096
    assert 0.6 < cache.compression_ratio() < 0.85
