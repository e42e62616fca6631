"""CPU checks of the drop-in host API (no GPU needed).

- compress() writes the reference's container layout and header fields, with
  its routing: tied (md5, >= 1024 B) -> tied_ref, tiny (< 512 B) -> raw, bf16 ->
  bf16_chunked_v1, fp8 -> fp8_chunked_v1, other dtypes -> raw; every blob's
  bytes decode (through the oracle's CPU decoder of the GPU format) to the
  source tensor's bytes, and match the header md5;
- codec_registry keeps the reference's plugin API and smallest-wins rule;
- the KV entry framing (versions 1/2 refused, version 3 parsed);
- StreamingLoader's index (layers, shards, duplicate_map) builds without a GPU;
- without a GPU, every decode entry point raises instead of decoding on the CPU.
"""
from __future__ import annotations

import hashlib
import json

import numpy as np
import pytest
import torch

import oracle
from bigsmall_amd import codec_registry, container, engine, kernels
from bigsmall_amd.codecs import kv_cache
from bigsmall_amd.encoder import compress
from bigsmall_amd.exceptions import BigSmallVersionError
from bigsmall_amd.streaming import StreamingLoader, layer_index
from bigsmall_amd.verify import verify_fast


def _model(seed=0, layers=2):
    g = torch.Generator().manual_seed(seed)
    t = {}
    for i in range(layers):
        p = f"model.layers.{i}."
        t[p + "self_attn.q_proj.weight"] = (torch.randn(256, 128, generator=g) * 0.02).bfloat16()
        t[p + "mlp.up_proj.weight"] = (torch.randn(300, 128, generator=g) * 0.02).bfloat16()
        t[p + "input_layernorm.weight"] = (1 + torch.randn(128, generator=g) * 0.01).bfloat16()
        t[p + "self_attn.q_proj.bias"] = torch.zeros(16, dtype=torch.bfloat16)           # tiny -> raw
    t["model.embed_tokens.weight"] = (torch.randn(512, 128, generator=g) * 0.02).bfloat16()
    t["lm_head.weight"] = t["model.embed_tokens.weight"].clone()                         # tied
    t["model.norm.weight"] = torch.ones(128, dtype=torch.bfloat16)
    t["fp8.weight"] = torch.randn(4096, generator=g).to(torch.float8_e4m3fn)
    t["f32.weight"] = torch.randn(300, generator=g)
    t["position_ids"] = torch.arange(1000, dtype=torch.int64)
    return t


@pytest.fixture(scope="module")
def container_file(tmp_path_factory):
    oracle.build()
    p = tmp_path_factory.mktemp("bs") / "m.bs"
    src = _model()
    compress(src, p)
    return p, src


def test_container_fields_and_routing(container_file):
    p, src = container_file
    header, data_offset = container.read_header(p)
    assert header["_format_version"] == 2 and header["tensor_count"] == len(src)
    for k in ("format", "mode", "model_type", "base_model", "tensors", "codec_stats"):
        assert k in header
    by = {t["name"]: t for t in header["tensors"]}
    assert by["lm_head.weight"]["codec"] == "tied_ref"
    assert by["lm_head.weight"]["extra"]["tied_to"] == "model.embed_tokens.weight"
    assert by["model.layers.0.self_attn.q_proj.bias"]["codec"] == "raw"
    assert by["model.layers.0.self_attn.q_proj.weight"]["codec"] == "bf16_chunked_v1"
    assert by["fp8.weight"]["codec"] == "fp8_chunked_v1"
    assert by["f32.weight"]["codec"] == "raw" and by["position_ids"]["codec"] == "raw"
    for t in header["tensors"]:
        assert set(t) >= {"name", "shape", "dtype", "codec", "special", "compressed_bytes", "offset", "md5", "extra"}
        if t["codec"] not in ("tied_ref", "raw"):
            assert t["offset"] % 256 == 0


def test_blobs_decode_to_source_via_oracle(container_file):
    p, src = container_file
    header, data_offset = container.read_header(p)
    for i, t in enumerate(header["tensors"]):
        want = src[t["name"]].contiguous().view(torch.uint8).numpy().tobytes()
        assert hashlib.md5(want).hexdigest() == t["md5"]
        blob = container.read_blob(p, header, data_offset, i)
        if t["codec"] == "raw":
            assert blob == want
        elif t["codec"] in ("bf16_chunked_v1", "fp8_chunked_v1"):
            eb = 2 if t["codec"] == "bf16_chunked_v1" else 1
            assert oracle.chunk_decode(blob, len(want) // eb, eb) == want, t["name"]


def test_info_and_verify_fast(container_file):
    p, _ = container_file
    inf = container.info(p)
    assert inf["layer_count"] == 2 and inf["tensor_count"] == inf["tensor_count"]
    ok, problems = verify_fast(p)
    assert ok, problems


def test_unsupported_codec_raises_version_error():
    for codec in ["bf16_se_rans", "bf16_se_ac", "fp8_cat_ac", "special", "something_new"]:
        with pytest.raises(BigSmallVersionError):
            engine.check_supported({"codec": codec, "name": "x"})
    with pytest.raises(BigSmallVersionError, match="blosc2"):
        engine.check_supported({"codec": "special", "name": "x", "extra": {"special_kind": "wpe_delta"}})
    for codec in ["raw", "tied_ref", "bf16_chunked_v1", "bf16_parallel_v1", "bf16_se_tans", "bf16_se_single_kernel",
                  "zstd", "zstd_xor_delta"]:
        engine.check_supported({"codec": codec, "name": "x"})
    engine.check_supported({"codec": "special", "name": "x", "extra": {"special_kind": "lowcard"}})


def test_registry_plugin_api_and_smallest_wins(monkeypatch):
    assert codec_registry.get_codec("bf16_chunked_v1") is not None
    calls = []

    def fake_enc(raw, **_):
        calls.append(1)
        return b"x", {"fake": True}

    codec_registry.register_codec("fake_small", fake_enc, lambda b, e, n: b"")
    monkeypatch.setitem(codec_registry.CODEC_CANDIDATES, "bf16", ["bf16_chunked_v1", "fake_small"])
    raw = (torch.randn(10000) * 0.02).bfloat16().view(torch.uint8).numpy().tobytes()
    blob, name, extras = codec_registry.auto_select_codec(raw, "bf16", "bfloat16")
    assert name == "fake_small" and blob == b"x" and calls
    # failing candidates are skipped, never raised
    codec_registry.register_codec("broken", lambda raw, **_: 1 / 0, lambda *a: b"")
    monkeypatch.setitem(codec_registry.CODEC_CANDIDATES, "bf16", ["broken"])
    blob, name, _ = codec_registry.auto_select_codec(raw, "bf16", "bfloat16")
    assert name == "raw" and blob == raw


def test_kv_entry_framing():
    k = (torch.randn(1, 4, 64, 32) * 2).bfloat16()
    v = (torch.randn(1, 4, 64, 32) * 0.5).bfloat16()
    data = kv_cache.compress_kv_entry(k, v)
    assert data[0] == 3
    parts = kv_cache.parse_kv_entry(data)
    for (shape, n, off, blen), t in zip(parts, (k, v)):
        assert shape == list(t.shape) and n == t.numel()
        want = t.view(torch.int16).numpy().view(np.uint16).tobytes()
        assert oracle.chunk_decode(data[off:off + blen], n) == want
    for ver in (1, 2):
        with pytest.raises(BigSmallVersionError):
            kv_cache.parse_kv_entry(bytes([ver]) + data[1:])


@pytest.mark.parametrize("shape,td,bt", [((8, 1024, 128), 1, 256), ((2, 8, 512, 64), 2, 128),
                                         ((8, 128, 1024), 2, 256), ((3, 1024, 6), 1, 256)])
def test_block_major_copy_matches_movedim(shape, td, bt):
    """The KV block split (copied as 8-byte words where the innermost
    dimension allows) gives exactly movedim(token-block dim, 0).contiguous()."""
    from bigsmall_amd.kv_cache_manager import _block_major
    t = torch.randn(shape, generator=torch.Generator().manual_seed(len(shape))).bfloat16()
    b = t.reshape(list(shape[:td]) + [shape[td] // bt, bt] + list(shape[td + 1:]))
    got, want = _block_major(b, td), b.movedim(td, 0).contiguous()
    assert got.dtype == want.dtype and got.shape == want.shape
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_streaming_index_without_gpu(container_file, tmp_path):
    p, src = container_file
    with StreamingLoader(p) as L:
        assert L.layer_count() == 2
        assert set(L.layer_tensor_names(0)) == {n for n in src if layer_index(n) == 0}
        assert "lm_head.weight" in L.non_layer_tensor_names()
    # directory with an index and a duplicate_map alias
    d = tmp_path / "sharded"
    d.mkdir()
    (d / "a.bs").write_bytes(p.read_bytes())
    (d / "bigsmall.index.json").write_text(json.dumps(
        {"metadata": {"shards": ["a.bs"], "duplicate_map": {"alias.weight": {"master": "model.norm.weight"}}}}))
    with StreamingLoader(d) as L:
        assert "alias.weight" in L.tensor_names()


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
def test_no_cpu_fallback(container_file):
    from bigsmall_amd import decoder
    p, _ = container_file
    kernels._GPU_BACKEND = None
    assert not kernels.use_gpu() and kernels.backend_name() == "cpu"
    with pytest.raises(RuntimeError):
        kernels.decode_bf16_parallel(b"PAR1xxxx", {}, 10)
    with pytest.raises(RuntimeError):
        decoder.load(p)


def test_kv_compression_ratio_below_75pct():
    """Mirror of the reference's KV ratio gate (tests/test_kv_cache.py:34-49):
    Gaussian KV-shaped tensors compress below 75 % of raw (host encoder)."""
    from bigsmall_amd.kv_cache_manager import CompressedKVCache
    torch.manual_seed(0)
    B, H, T, D = 1, 32, 512, 96
    k = (torch.randn(B, H, T, D) * 0.5).to(torch.bfloat16)
    v = (torch.randn(B, H, T, D) * 0.5).to(torch.bfloat16)
    raw = k.element_size() * k.numel() + v.element_size() * v.numel()
    ratio = len(kv_cache.compress_kv_entry(k, v)) / raw
    assert ratio < 0.75, f"KV compression ratio {ratio * 100:.2f}% exceeds the 75% gate"
    cache = CompressedKVCache(device="cuda")       # the empty-cache API needs no GPU
    assert len(cache) == 0 and cache.memory_usage() == 0 and cache.compression_ratio() is None


def test_kv_len_counts_a_layer_once_and_block_ids_are_checked():
    """A layer stored through set() and set_blocks() counts once; a negative
    or too-large block id raises IndexError instead of wrapping."""
    from bigsmall_amd.kv_cache_manager import CompressedKVCache, _LayerBlocks
    torch.manual_seed(1)
    k = (torch.randn(1, 2, 64, 8) * 0.5).to(torch.bfloat16)
    cache = CompressedKVCache(device="cuda")
    cache.set(0, k, k)
    cache._blocks[0] = _LayerBlocks([1, 2, 16, 8], 256, None, [(0, 16, 1, 1)] * 4, [(0, 16, 1, 1)] * 4)
    cache._blocks[1] = cache._blocks[0]
    assert len(cache) == 2
    L = cache._blocks[0]
    assert cache._block_ids(L, 0, [0, 3, 2]) == [0, 3, 2]
    for bad in ([-1], [4], [0, 7]):
        with pytest.raises(IndexError):
            cache._block_ids(L, 0, bad)


@pytest.mark.parametrize("master_dtype,follower_dtype,shape", [
    (torch.float32, torch.int32, [4, 300]),          # all-zero buffers of two dtypes share one blob
    (torch.bfloat16, torch.float16, [600]),          # same 16-bit words, other dtype
    (torch.bfloat16, torch.bfloat16, [20, 30]),      # same dtype and shape: a plain copy
    (torch.bfloat16, torch.bfloat16, [600]),         # same bytes, other shape
])
def test_tied_follower_takes_its_own_dtype_and_shape(master_dtype, follower_dtype, shape):
    """The engine's tied copy reinterprets the master's bytes with the
    follower's dtype and shape, as the reference's _raw_to_numpy does with the
    master's raw bytes (bigsmall/decoder.py:138-155)."""
    g = torch.Generator().manual_seed(3)
    words = torch.randint(0, 1 << 15, (600,), generator=g, dtype=torch.int16)
    master = words.view(master_dtype) if master_dtype != torch.float32 else torch.zeros(1200, dtype=torch.float32)
    master = master.reshape(20, 30) if master.numel() == 600 else master.reshape(4, 300)
    t = {"name": "f", "dtype": {torch.int32: "I32", torch.float16: "F16", torch.bfloat16: "BF16"}[follower_dtype],
         "shape": shape}
    out = engine.tied_copy(master, t)
    assert out.dtype == follower_dtype and list(out.shape) == shape
    assert out.contiguous().view(-1).view(torch.uint8).tolist() == master.contiguous().view(-1).view(torch.uint8).tolist()
    assert out.data_ptr() != master.data_ptr()
    with pytest.raises(ValueError):
        engine.tied_copy(master, {**t, "shape": [7]})


def test_streaming_gpt2_block_math_matches_transformers():
    """StreamingGPT2's block (bigsmall/streaming_model.py:84-132), fed the
    uncompressed weights on the CPU, gives transformers' GPT2LMHeadModel
    logits to 1e-4 and the same greedy tokens."""
    from transformers import GPT2Config, GPT2LMHeadModel
    from bigsmall_amd.streaming_model import StreamingGPT2

    class DictLoader:
        def __init__(self, sd):
            self.sd = sd

        def load_non_layer_tensors(self):
            return {k: v for k, v in self.sd.items() if not k.startswith("h.")}

        def iter_layers(self, progress=True):
            for i in range(3):
                yield i, {k: v for k, v in self.sd.items() if k.startswith(f"h.{i}.")}

    cfg = GPT2Config(n_layer=3, n_embd=64, n_head=4, vocab_size=300, n_positions=64, bos_token_id=0, eos_token_id=0)
    torch.manual_seed(0)
    model = GPT2LMHeadModel(cfg).eval()
    with torch.no_grad():
        for prm in model.parameters():        # weights large enough that logits have clear margins
            prm.mul_(8.0)
    sd = {k[len("transformer."):]: v.detach().clone() for k, v in model.state_dict().items()
          if k.startswith("transformer.")}
    sm = StreamingGPT2(DictLoader(sd), config=cfg, device="cpu")
    ids = torch.randint(0, 300, (2, 11), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        hf = model(ids).logits
    assert torch.allclose(sm.forward(ids), hf, atol=1e-4, rtol=1e-4)
    with torch.no_grad():
        hf_gen = model.generate(input_ids=ids[:1], max_new_tokens=4, do_sample=False, pad_token_id=0)
    assert torch.equal(sm.generate_greedy(ids[:1], 4), hf_gen)
