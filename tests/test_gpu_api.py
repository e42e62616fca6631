"""GPU tests of the drop-in API: decoder.load / decompress / _decode_blob,
verify, StreamingLoader (with and without prefetch), containers mixing the
engine's format with the reference's formats, CompressedKVCache entries and
blocks, and BigSmallStreamingModel against a normally loaded model.

Bar: bit-exact (every decoded tensor's bytes equal the source's).
"""
from __future__ import annotations

import hashlib
import sys

import numpy as np
import pytest
import torch

import oracle
from bigsmall_amd import container
from bigsmall_amd.encoder import compress

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _bytes(t):
    return t.detach().contiguous().cpu().view(torch.uint8).numpy().tobytes()


def _model(seed=0, layers=3, width=256):
    g = torch.Generator().manual_seed(seed)
    t = {}
    for i in range(layers):
        p = f"model.layers.{i}."
        t[p + "self_attn.q_proj.weight"] = (torch.randn(width, width, generator=g) * 0.02).bfloat16()
        t[p + "self_attn.k_proj.weight"] = (torch.randn(width // 4, width, generator=g) * 0.02).bfloat16()
        t[p + "mlp.down_proj.weight"] = (torch.randn(width, 3 * width + 5, generator=g) * 0.02).bfloat16()
        t[p + "input_layernorm.weight"] = (1 + torch.randn(width, generator=g) * 0.01).bfloat16()
        t[p + "self_attn.q_proj.bias"] = torch.zeros(16, dtype=torch.bfloat16)
    t["model.embed_tokens.weight"] = (torch.randn(1000, width, generator=g) * 0.02).bfloat16()
    t["lm_head.weight"] = t["model.embed_tokens.weight"].clone()
    t["model.norm.weight"] = torch.ones(width, dtype=torch.bfloat16)
    t["fp8.weight"] = torch.randn(70_000, generator=g).to(torch.float8_e4m3fn)
    t["f32.weight"] = torch.randn(3000, generator=g)
    t["steps"] = torch.arange(10, dtype=torch.int64)
    return t


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    assert torch.cuda.is_available()
    oracle.build()
    p = tmp_path_factory.mktemp("bs") / "m.bs"
    src = _model()
    compress(src, p)
    return p, src


def test_load_decompress_verify(model_file):
    from bigsmall_amd import decoder
    from bigsmall_amd.verify import verify
    p, src = model_file
    _say("[api] load")
    dev = decoder.load(p, device="cuda")
    assert list(dev) == list(src)
    for k, v in src.items():
        assert dev[k].device.type == "cuda" and dev[k].dtype == v.dtype and tuple(dev[k].shape) == tuple(v.shape)
        assert _bytes(dev[k]) == _bytes(v), k
    _say("[api] decompress")
    host = decoder.decompress(p)
    header, _ = container.read_header(p)
    for t in header["tensors"]:
        assert hashlib.md5(host[t["name"]].tobytes()).hexdigest() == t["md5"], t["name"]
    assert verify(p)
    cpu = decoder.load(p, device="cpu")
    assert all(_bytes(cpu[k]) == _bytes(src[k]) for k in src)


def test_decode_blob_each_codec(model_file):
    from bigsmall_amd import decoder
    p, src = model_file
    header, off = container.read_header(p)
    for i, t in enumerate(header["tensors"]):
        raw = decoder._decode_blob(t, container.read_blob(p, header, off, i))
        if t["codec"] == "tied_ref":
            assert raw is None
        else:
            assert raw == _bytes(src[t["name"]]), t["name"]


def _write_mixed(path, align_odd=True):
    """Container with reference-format blobs (oracle encoders = reference bytes)
    and one BSCK blob at an offset that is not 16-byte aligned."""
    from bigsmall_amd.codecs import bf16_chunked
    rng = np.random.default_rng(3)

    def words(n, s=0.02):
        x = (rng.standard_normal(n) * s).astype(np.float32).view(np.uint32).astype(np.uint64)
        return ((x + 0x7FFF + ((x >> 16) & 1)) >> 16).astype(np.uint16)

    items = [("model.layers.0.a.weight", words(120_000), "bf16_parallel_v1", oracle.par1_encode),
             ("model.layers.0.b.weight", words(50_001), "bf16_se_tans", oracle.tans_encode),
             ("model.layers.1.c.weight", words(77_777), "bf16_se_single_kernel", oracle.sk_encode),
             ("model.layers.1.d.weight", words(200_000), "bf16_chunked_v1", lambda w: bf16_chunked.encode_array(w))]
    data, tensors = bytearray(), []
    for name, w, codec, enc in items:
        if align_odd:
            data += b"\x00" * 3
        blob = enc(w)
        tensors.append({"name": name, "shape": [w.size], "dtype": "bfloat16", "codec": codec, "special": None,
                        "compressed_bytes": len(blob), "offset": len(data),
                        "md5": hashlib.md5(w.tobytes()).hexdigest(), "extra": None})
        data += blob
    header = {"format": "bf16", "mode": "balanced", "model_type": "llm", "base_model": None,
              "tensor_count": len(tensors), "tensors": tensors}
    container.write_container(path, header, bytes(data), format_version=2)
    return {name: w for name, w, _, _ in items}


def test_mixed_reference_formats_and_misaligned_blobs(tmp_path):
    from bigsmall_amd import decoder
    from bigsmall_amd.streaming import StreamingLoader
    p = tmp_path / "mixed.bs"
    src = _write_mixed(p)
    _say("[api] mixed container load")
    out = decoder.load(p)
    for k, w in src.items():
        assert out[k].view(torch.int16).cpu().numpy().view(np.uint16).tobytes() == w.tobytes(), k
    with StreamingLoader(p) as L:
        for li, layer in L.iter_layers():
            for k, t in layer.items():
                assert t.view(torch.int16).cpu().numpy().view(np.uint16).tobytes() == src[k].tobytes()


def test_pruned_tensors_written_as_table_ans_load_bit_exact(tmp_path):
    """compress() gives a large half-pruned tensor the table-ANS form
    (auto-selection's compact-tANS rule) and a dense one rANS; both come back
    bit-exact through decoder.load (one batched launch per layer group, both
    coders in it), decompress, verify and the streaming loader."""
    from bigsmall_amd import decoder
    from bigsmall_amd.codecs import bf16_chunked as bc
    from bigsmall_amd.streaming import StreamingLoader
    from bigsmall_amd.verify import verify
    g = torch.Generator().manual_seed(31)
    pruned = (torch.randn(4096, 1024, generator=g) * 0.02).bfloat16()
    pruned.view(-1)[torch.randperm(pruned.numel(), generator=g)[: pruned.numel() // 2]] = 0
    src = {"model.layers.0.mlp.down_proj.weight": pruned,
           "model.layers.0.self_attn.q_proj.weight": (torch.randn(1024, 1024, generator=g) * 0.02).bfloat16(),
           "model.layers.1.mlp.down_proj.weight": pruned.flip(0).contiguous()}
    p = tmp_path / "pruned.bs"
    _say("[api] compress a pruned layer")
    compress(src, p)
    header, _ = container.read_header(p)
    codecs = {t["name"]: t["codec"] for t in header["tensors"]}
    assert codecs["model.layers.0.mlp.down_proj.weight"] == bc.CODEC_BF16_TANS
    assert codecs["model.layers.1.mlp.down_proj.weight"] == bc.CODEC_BF16_TANS
    assert codecs["model.layers.0.self_attn.q_proj.weight"] == bc.CODEC_BF16
    _say("[api] load / decompress / verify the pruned layer")
    dev = decoder.load(p, device="cuda")
    assert all(_bytes(dev[k]) == _bytes(v) for k, v in src.items())
    host = decoder.decompress(p)
    assert all(host[k].tobytes() == _bytes(v) for k, v in src.items())
    assert verify(p)
    with StreamingLoader(p, device="cuda", prefetch=1) as L:
        for li, layer in L.iter_layers():
            for k, t in layer.items():
                assert _bytes(t) == _bytes(src[k]), k


@pytest.mark.parametrize("prefetch", [0, 1, 2])
def test_streaming_loader(model_file, prefetch):
    from bigsmall_amd.streaming import StreamingLoader
    p, src = model_file
    _say(f"[api] streaming prefetch={prefetch}")
    with StreamingLoader(p, device="cuda", prefetch=prefetch) as L:
        seen = set()
        for li, layer in L.iter_layers():
            assert set(layer) == set(L.layer_tensor_names(li))
            for k, t in layer.items():
                assert _bytes(t) == _bytes(src[k]), k
                seen.add(k)
        assert len(seen) == sum(1 for k in src if k.startswith("model.layers."))
        nl = L.load_non_layer_tensors()
        assert _bytes(nl["lm_head.weight"]) == _bytes(src["model.embed_tokens.weight"])
        assert _bytes(L.load_tensor("model.layers.1.mlp.down_proj.weight")) == \
            _bytes(src["model.layers.1.mlp.down_proj.weight"])
        lay = L.load_layer(2)
        assert all(_bytes(v) == _bytes(src[k]) for k, v in lay.items())
    with StreamingLoader(p, dtype=torch.float32) as L:
        lay = L.load_layer(0)
        assert lay["model.layers.0.self_attn.q_proj.weight"].dtype == torch.float32
        assert torch.equal(lay["model.layers.0.self_attn.q_proj.weight"].cpu(),
                           src["model.layers.0.self_attn.q_proj.weight"].float())


@pytest.mark.parametrize("prefetch", [0, 1])
def test_streaming_loader_reports_a_corrupt_layer(model_file, tmp_path, prefetch):
    """A renorm word flipped inside layer 1's q_proj blob: loading layer 1
    raises DecodeError on the caller's thread (also when the decode ran on the
    loader's worker thread), and the same loader still decodes the other
    layers bit-exactly afterwards."""
    from bigsmall_amd.exceptions import DecodeError
    from bigsmall_amd.streaming import StreamingLoader
    p, src = model_file
    header, data_offset = container.read_header(p)
    t = next(x for x in header["tensors"] if x["name"] == "model.layers.1.self_attn.q_proj.weight")
    assert t["codec"] == "bf16_chunked_v1"
    raw = bytearray(p.read_bytes())
    blob0 = data_offset + int(t["offset"])
    nsym = int.from_bytes(raw[blob0 + 22:blob0 + 24], "little")
    ctab = (32 + 4 * nsym + 15) & ~15
    c0 = int.from_bytes(raw[blob0 + ctab:blob0 + ctab + 8], "little")
    lanes = int.from_bytes(raw[blob0 + 20:blob0 + 22], "little")
    raw[blob0 + c0 + 4 * lanes + 6] ^= 0x5A             # a renorm word of chunk 0
    bad = tmp_path / "bad.bs"
    bad.write_bytes(bytes(raw))
    _say(f"[api] corrupt layer 1, prefetch={prefetch}")
    with StreamingLoader(bad, device="cuda", prefetch=prefetch) as L:
        with pytest.raises(DecodeError):
            L.load_layer(1)
        for li in (0, 2):
            lay = L.load_layer(li)
            assert all(_bytes(v) == _bytes(src[k]) for k, v in lay.items()), li


def test_kv_cache_entries_and_blocks():
    from bigsmall_amd.kv_cache_manager import CompressedKVCache
    g = torch.Generator().manual_seed(9)
    scale = torch.empty(1, 8, 1, 1).uniform_(0.5, 2.0, generator=g)
    k = (torch.randn(1, 8, 1024, 128, generator=g) * scale).bfloat16()
    v = (torch.randn(1, 8, 1024, 128, generator=g) * scale).bfloat16()
    c = CompressedKVCache(device="cuda")
    c.set(0, k, v)
    kk, vv = c.get(0)
    assert _bytes(kk) == _bytes(k) and _bytes(vv) == _bytes(v)
    assert 0.6 < c.compression_ratio() < 0.9
    K, V = k[0], v[0]                                   # [8 heads, 1024 tokens, 128]
    nb = c.set_blocks(1, K, V, block_tokens=256)
    assert nb == 4
    ids = [3, 0, 2, 2]
    _say("[api] kv blocks")
    kb, vb = c.get_blocks(1, ids)
    for j, b in enumerate(ids):
        assert _bytes(kb[j]) == _bytes(K[:, b * 256:(b + 1) * 256, :]), j
        assert _bytes(vb[j]) == _bytes(V[:, b * 256:(b + 1) * 256, :]), j
    c.set_blocks(2, V, K, block_tokens=256)
    (k1, v1), (k2, v2) = c.get_blocks_multi([(1, [1]), (2, [0, 3])])
    assert _bytes(k1[0]) == _bytes(K[:, 256:512]) and _bytes(k2[1]) == _bytes(V[:, 768:1024])
    assert _bytes(v2[0]) == _bytes(K[:, 0:256])


def _md5_tensor(t) -> str:
    return hashlib.md5(t.contiguous().view(torch.uint8).cpu().numpy().tobytes()).hexdigest()


@pytest.mark.parametrize("device", ["cuda", "cpu"])
def test_reference_kv_cache_tests(device):
    """Mirrors of the reference's KV-cache tests (tests/test_kv_cache.py:15-119):
    entry round trip, CompressedKVCache set/get/has/len/memory_usage/
    compression_ratio, several layers, clear(). Decoding runs on the GPU; with
    device="cpu" the tensors come back to host memory."""
    from bigsmall_amd.codecs.kv_cache import compress_kv_entry, decompress_kv_entry
    from bigsmall_amd.kv_cache_manager import CompressedKVCache
    _say(f"[api] reference KV tests, device={device}")
    torch.manual_seed(0)
    k = torch.randn(1, 32, 64, 96, dtype=torch.float32).to(torch.bfloat16)
    v = torch.randn(1, 32, 64, 96, dtype=torch.float32).to(torch.bfloat16)
    k2, v2 = decompress_kv_entry(compress_kv_entry(k, v), device=device)
    assert k2.device.type == device and v2.device.type == device
    assert _md5_tensor(k) == _md5_tensor(k2) and _md5_tensor(v) == _md5_tensor(v2)

    torch.manual_seed(1)
    cache = CompressedKVCache(device=device)
    assert len(cache) == 0 and cache.memory_usage() == 0 and cache.compression_ratio() is None
    k = torch.randn(1, 32, 64, 96).to(torch.bfloat16)
    v = torch.randn(1, 32, 64, 96).to(torch.bfloat16)
    cache.set(0, k, v)
    assert cache.has(0) and len(cache) == 1
    k2, v2 = cache.get(0)
    assert _md5_tensor(k) == _md5_tensor(k2) and _md5_tensor(v) == _md5_tensor(v2)
    cr = cache.compression_ratio()
    assert cr is not None and 0.0 < cr < 1.0 and cache.memory_usage() > 0

    cache = CompressedKVCache(device=device)
    layers = {}
    torch.manual_seed(2)
    for li in range(4):
        layers[li] = (torch.randn(1, 32, 32, 96).to(torch.bfloat16), torch.randn(1, 32, 32, 96).to(torch.bfloat16))
        cache.set(li, *layers[li])
    for li in range(4):
        k2, v2 = cache.get(li)
        assert _md5_tensor(layers[li][0]) == _md5_tensor(k2) and _md5_tensor(layers[li][1]) == _md5_tensor(v2), li

    cache.clear()
    assert len(cache) == 0 and cache.memory_usage() == 0 and cache.compression_ratio() is None


def test_reference_bf16_parallel_lossless_gaussian():
    """Mirror of the reference's tests/test_bf16_parallel.py:27-36: n = 2^20
    N(0, 0.02) bf16 words, N in {1, 32, 128, 256} streams, decoded through the
    plugin decode(blob, extras, n) on the GPU (blobs from the oracle's encoder,
    byte-identical to the reference's on the golden vectors)."""
    from bigsmall_amd.codecs import bf16_parallel
    torch.manual_seed(0)
    n = 1 << 20
    raw = (torch.randn(n) * 0.02).to(torch.bfloat16).view(torch.uint8).numpy().tobytes()
    words = np.frombuffer(raw, np.uint16)
    for ns in [1, 32, 128, 256]:
        _say(f"[api] bf16_parallel_v1 n=2^20 N={ns}")
        out = bf16_parallel.decode(oracle.par1_encode(words, ns), {}, n)
        assert hashlib.md5(raw).hexdigest() == hashlib.md5(out).hexdigest(), f"mismatch at N={ns}"


def test_reference_bf16_parallel_edge_cases():
    """Mirror of tests/test_bf16_parallel.py:39-62: NaN, +/-Inf, +/-0, the
    smallest denormal and normal, 1.0, then 4096 normals, N in {1, 32, 128}."""
    import struct
    from bigsmall_amd.codecs import bf16_parallel
    special = [0x7FC0, 0x7F80, 0xFF80, 0x0000, 0x8000, 0x0001, 0x0080, 0x3F80]
    torch.manual_seed(1)
    normals = (torch.randn(4096) * 0.02).to(torch.bfloat16).view(torch.uint8).numpy()
    raw = b"".join(struct.pack("<H", w) for w in special) + normals.tobytes()
    n = len(raw) // 2
    for ns in [1, 32, 128]:
        out = bf16_parallel.decode(oracle.par1_encode(np.frombuffer(raw, np.uint16), ns), {}, n)
        assert raw == out, f"byte mismatch at N={ns}"


def test_reference_streaming_md5_roundtrip_all_layers(tmp_path):
    """Mirror of tests/test_streaming.py:38-127: a synthetic 4-layer model
    (embed, ln_f, q/k/up/down projections and a norm per layer, N(0, 1) bf16)
    through compress_for_hub, then StreamingLoader on the output directory:
    layer count, the non-layer names, and every tensor md5-equal to its source,
    from load_non_layer_tensors and iter_layers (device="cpu": decoded on the
    GPU, returned in host memory)."""
    from safetensors.torch import save_file
    import bigsmall_amd
    from bigsmall_amd.streaming import StreamingLoader, layer_index
    n_layers, hidden = 4, 256
    torch.manual_seed(0)
    src = {"embed.weight": torch.randn(1024, hidden, dtype=torch.bfloat16),
           "ln_f.weight": torch.randn(hidden, dtype=torch.bfloat16),
           "ln_f.bias": torch.zeros(hidden, dtype=torch.bfloat16)}
    for i in range(n_layers):
        p = f"model.layers.{i}"
        src[f"{p}.self_attn.q_proj.weight"] = torch.randn(hidden, hidden, dtype=torch.bfloat16)
        src[f"{p}.self_attn.k_proj.weight"] = torch.randn(hidden, hidden, dtype=torch.bfloat16)
        src[f"{p}.mlp.up_proj.weight"] = torch.randn(hidden * 2, hidden, dtype=torch.bfloat16)
        src[f"{p}.mlp.down_proj.weight"] = torch.randn(hidden, hidden * 2, dtype=torch.bfloat16)
        src[f"{p}.input_layernorm.weight"] = torch.randn(hidden, dtype=torch.bfloat16)
    (tmp_path / "src").mkdir()
    save_file(src, str(tmp_path / "src" / "model.safetensors"))
    out = tmp_path / "out"
    bigsmall_amd.compress_for_hub(str(tmp_path / "src"), output_dir=out, overwrite=True)
    want = {k: _md5_tensor(v) for k, v in src.items()}
    seen = set()
    with StreamingLoader(str(out), device="cpu") as L:
        assert L.layer_count() == n_layers
        assert sorted(L.non_layer_tensor_names()) == ["embed.weight", "ln_f.bias", "ln_f.weight"]
        for name, t in L.load_non_layer_tensors().items():
            seen.add(name)
            assert _md5_tensor(t) == want[name], name
        for li, layer in L.iter_layers():
            for name, t in layer.items():
                seen.add(name)
                assert layer_index(name) == li and t.device.type == "cpu"
                assert _md5_tensor(t) == want[name], name
    assert seen == set(want)


def test_reference_decompress_layers_returns_only_requested(tmp_path):
    """Mirror of tests/test_opt_step6.py:93-135: decompress_layers returns the
    requested layers only (equal to the source), non-layer tensors only on
    request, and a missing layer raises ValueError."""
    import bigsmall_amd
    torch.manual_seed(2)
    sd = {"model.embed_tokens.weight": (torch.randn(1024, 64) * 0.02).to(torch.bfloat16)}
    for i in range(6):
        sd[f"model.layers.{i}.q.weight"] = (torch.randn(64, 64) * 0.02).to(torch.bfloat16)
        sd[f"model.layers.{i}.k.weight"] = (torch.randn(64, 64) * 0.02).to(torch.bfloat16)
    sd["model.norm.weight"] = (torch.randn(64) * 0.02).to(torch.bfloat16)
    bs = tmp_path / "model.bs"
    compress(sd, bs)
    partial = bigsmall_amd.decompress_layers(bs, layer_indices=[1, 3], device="cpu")
    assert set(partial) == {f"model.layers.{li}.{w}.weight" for li in (1, 3) for w in ("q", "k")}
    for k, v in partial.items():
        assert v.device.type == "cpu" and _bytes(v) == _bytes(sd[k]), k
    with_extras = bigsmall_amd.decompress_layers(bs, layer_indices=[0], device="cuda", include_non_layer=True)
    assert {"model.embed_tokens.weight", "model.norm.weight", "model.layers.0.q.weight"} <= set(with_extras)
    assert _bytes(with_extras["model.embed_tokens.weight"]) == _bytes(sd["model.embed_tokens.weight"])
    with pytest.raises(ValueError):
        bigsmall_amd.decompress_layers(bs, layer_indices=[7])


def test_streaming_model_matches_full_model(tmp_path):
    """A tiny Llama decoded layer by layer gives the same logits as the same
    weights loaded whole (float32 compute)."""
    from transformers import LlamaConfig, LlamaForCausalLM
    from bigsmall_amd.streaming_inference import BigSmallStreamingModel
    cfg = LlamaConfig(vocab_size=256, hidden_size=128, intermediate_size=320, num_hidden_layers=3,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
                      tie_word_embeddings=False, attn_implementation="eager")
    torch.manual_seed(0)
    ref = LlamaForCausalLM(cfg)            # float32 module; weights rounded to bf16 values
    with torch.no_grad():
        for prm in ref.parameters():
            prm.copy_(prm.bfloat16().float())
    sd = {k: v.bfloat16().contiguous() for k, v in ref.state_dict().items()}
    bs = tmp_path / "tiny.bs"
    compress(sd, bs)
    cfg.save_pretrained(tmp_path)
    ids = torch.randint(0, 256, (1, 12), generator=torch.Generator().manual_seed(1))
    ref = ref.cuda().eval()
    with torch.no_grad():
        want = ref(ids.cuda()).logits
    for prefetch in (0, 1):
        _say(f"[api] streaming model prefetch={prefetch}")
        m = BigSmallStreamingModel.from_pretrained(bs, device="cuda", dtype=torch.float32, prefetch=prefetch)
        for _ in range(2):                         # a second pass must prefetch too
            got = m.forward(ids.cuda()).logits
            diff = (got - want).abs().max().item()
            _say(f"[api]   max |logit diff| = {diff:.3e}")
            # the weights are bit-exact (tests above); fp32 GEMMs on separately
            # allocated parameters may pick other kernels, so allow rounding noise
            assert diff <= 1e-5 * max(1.0, want.abs().max().item())
            assert torch.equal(got.argmax(-1), want.argmax(-1))
        m.close()


def test_from_pretrained_multi_shard(tmp_path):
    """compress_for_hub over two safetensors shards with a cross-shard tied
    tensor, then from_pretrained decodes every shard on the GPU; the alias
    shares its master's tensor and every tensor is bit-exact."""
    import json as _json
    from safetensors.torch import save_file
    from bigsmall_amd import hub
    src = tmp_path / "src"
    src.mkdir()
    m = _model(seed=4, layers=4)
    emb = m.pop("model.embed_tokens.weight")
    m.pop("lm_head.weight")
    names = sorted(k for k in m if m[k].dtype == torch.bfloat16)
    a = {k: m[k] for k in names[: len(names) // 2]} | {"model.embed_tokens.weight": emb}
    b = {k: m[k] for k in names[len(names) // 2:]} | {"lm_head.weight": emb.clone()}
    save_file(a, str(src / "model-00001-of-00002.safetensors"))
    save_file(b, str(src / "model-00002-of-00002.safetensors"))
    wm = {k: "model-00001-of-00002.safetensors" for k in a} | {k: "model-00002-of-00002.safetensors" for k in b}
    (src / "model.safetensors.index.json").write_text(_json.dumps({"metadata": {}, "weight_map": wm}))
    out = tmp_path / "bs"
    hub.compress_for_hub(src, out)
    _say("[api] from_pretrained over 2 shards")
    sd = hub.from_pretrained(out, device="cuda")
    assert set(sd) == set(a) | set(b)
    for k, v in (a | b).items():
        assert _bytes(sd[k]) == _bytes(v), k
    assert sd["lm_head.weight"].data_ptr() == sd["model.embed_tokens.weight"].data_ptr()


def test_tie_across_dtypes_round_trip(tmp_path):
    """An all-zero F32 buffer and an all-zero I32 buffer of one shape, and BF16
    and F16 tensors holding the same 16-bit words, are tied by the encoder
    (item size, shape and md5 match, as in bigsmall/tensor_analysis.py:97-110);
    load(), decompress() and the streaming loader give each its own dtype."""
    from bigsmall_amd import decoder
    from bigsmall_amd.streaming import StreamingLoader
    g = torch.Generator().manual_seed(11)
    words = (torch.randn(64, 128, generator=g) * 0.02).bfloat16()
    src = {"model.layers.0.mlp.mask_f32": torch.zeros(8, 256, dtype=torch.float32),
           "model.layers.0.mlp.mask_i32": torch.zeros(8, 256, dtype=torch.int32),
           "model.layers.0.self_attn.w_bf16": words,
           "model.layers.0.self_attn.w_f16": words.view(torch.float16).clone(),
           "model.layers.1.self_attn.w_f16_2": words.view(torch.float16).clone()}
    p = tmp_path / "tied.bs"
    compress(src, p)
    header, _ = container.read_header(p)
    codecs = {t["name"]: t["codec"] for t in header["tensors"]}
    assert codecs["model.layers.0.mlp.mask_i32"] == "tied_ref" and codecs["model.layers.0.self_attn.w_f16"] == "tied_ref"
    _say("[api] tie across dtypes: load")
    out = decoder.load(p)
    for k, v in src.items():
        assert out[k].dtype == v.dtype and tuple(out[k].shape) == tuple(v.shape), k
        assert _bytes(out[k]) == _bytes(v), k
    host = decoder.decompress(p)
    for t in header["tensors"]:
        assert hashlib.md5(np.ascontiguousarray(host[t["name"]]).tobytes()).hexdigest() == t["md5"], t["name"]
    _say("[api] tie across dtypes: streaming")
    with StreamingLoader(p, prefetch=1) as L:
        got = {}
        for li, layer in L.iter_layers():
            got.update(layer)
    for k, v in src.items():
        assert got[k].dtype == v.dtype and _bytes(got[k]) == _bytes(v), k


class _DictLoader:
    """The two StreamingLoader calls StreamingGPT2 makes, served from a dict of
    uncompressed tensors: the same forward on the source weights."""

    def __init__(self, sd: dict, device):
        self.sd = {k: v.to(device) for k, v in sd.items()}

    def load_non_layer_tensors(self):
        return {k: v for k, v in self.sd.items() if not k.startswith("h.")}

    def iter_layers(self, progress=True):
        n = 1 + max(int(k.split(".")[1]) for k in self.sd if k.startswith("h."))
        for i in range(n):
            yield i, {k: v for k, v in self.sd.items() if k.startswith(f"h.{i}.")}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("prefetch", [0, 2])
def test_streaming_gpt2(tmp_path, dtype, prefetch):
    """StreamingGPT2 (bigsmall/streaming_model.py:29-176) over a random-init
    GPT-2-shaped model stored with the GPT-2 safetensors names: logits and
    greedy tokens equal the same forward on the uncompressed weights (the
    decoded weights are bit-exact), and in fp32 the logits agree with
    transformers' GPT2LMHeadModel to 1e-4."""
    from transformers import GPT2Config, GPT2LMHeadModel
    from bigsmall_amd.streaming import StreamingLoader
    from bigsmall_amd.streaming_model import StreamingGPT2
    cfg = GPT2Config(n_layer=3, n_embd=128, n_head=4, vocab_size=1000, n_positions=128, bos_token_id=0,
                     eos_token_id=0)
    torch.manual_seed(0)
    model = GPT2LMHeadModel(cfg).eval()
    sd = {k[len("transformer."):]: v.detach().clone().contiguous().to(dtype)
          for k, v in model.state_dict().items() if k.startswith("transformer.")}
    p = tmp_path / "gpt2.bs"
    compress(sd, p)
    ids = torch.randint(0, 1000, (2, 17), generator=torch.Generator().manual_seed(1))
    dev = torch.device("cuda", 0)
    _say(f"[api] StreamingGPT2 dtype={dtype} prefetch={prefetch}")
    ref = StreamingGPT2(_DictLoader(sd, dev), config=cfg, device="cuda")
    with StreamingLoader(p, device="cuda", prefetch=prefetch) as L:
        sm = StreamingGPT2(L, config=cfg, device="cuda")
        logits = sm.forward(ids)
        gen = sm.generate_greedy(ids[:1], max_new_tokens=5)
    want = ref.forward(ids)
    assert logits.dtype == dtype and torch.equal(logits, want)
    assert torch.equal(gen, ref.generate_greedy(ids[:1], max_new_tokens=5))
    if dtype == torch.float32:
        hf = model.to(dev)(ids.to(dev)).logits
        assert torch.allclose(logits, hf, atol=1e-4, rtol=1e-4), (logits - hf).abs().max()


@pytest.mark.parametrize("kw", [{"gpu_optimised": True}, {"prefer_speed": True}])
def test_compress_reference_formats_round_trip(tmp_path, kw):
    """Containers compress() writes with the reference's gpu_optimised /
    prefer_speed choices (bf16_parallel_v1, bf16_se_single_kernel or
    bf16_se_tans, by the reference's rules; lowcard tensors as `special`,
    other formats as `zstd`: only codecs the reference decodes) load
    bit-exactly on the GPU, one batched wave-serial launch per layer plus the
    GPU zstd decoder for the special and zstd entries."""
    from bigsmall_amd import decoder
    g = torch.Generator().manual_seed(12)
    src = {f"model.layers.{i}.mlp.{n}.weight": (torch.randn(2048, 2048 + 64 * i, generator=g) * 0.02).bfloat16()
           for i in range(2) for n in ("up_proj", "down_proj")}
    src["model.norm.weight"] = (1 + torch.randn(1024, generator=g) * 0.01).bfloat16()
    src["model.layers.0.attn.bias"] = torch.tril(torch.ones(128, 128)).bfloat16()
    src["model.layers.0.scale.f32"] = torch.randn(3000, generator=g)
    src["model.layers.0.ids"] = torch.arange(500, dtype=torch.int64)
    p = tmp_path / "ref_formats.bs"
    compress(src, p, **kw)
    header, _ = container.read_header(p)
    by = {t["name"]: t["codec"] for t in header["tensors"]}
    codecs = set(by.values())
    _say(f"[api] compress({kw}) codecs {sorted(codecs)}")
    assert codecs & {"bf16_parallel_v1", "bf16_se_single_kernel", "bf16_se_tans"}
    assert codecs <= {"bf16_parallel_v1", "bf16_se_single_kernel", "bf16_se_tans", "special", "zstd", "raw",
                      "tied_ref"}
    assert by["model.norm.weight"] == "special" and by["model.layers.0.ids"] == "zstd"
    out = decoder.load(p)
    for k, v in src.items():
        assert _bytes(out[k]) == _bytes(v), k
