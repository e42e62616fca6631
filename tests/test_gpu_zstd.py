"""GPU zstd decoding (bs_zstd_decode, bs_lut_expand) and the zstd-coded
container entries of the reference ("zstd", "special" lowcard).

Bar: bit-exact. Every frame decodes on the GPU to its source bytes, which
libzstd (the oracle) also returns for it. The frames cover raw, RLE and
compressed blocks; Huffman literals in one and four streams, with new and
repeated trees; predefined, RLE, FSE-coded and repeated sequence tables;
matches reaching across blocks; levels -5 to 22; content checksums; frames
with no content size; skippable and back-to-back frames. Corrupted frames
either decode to what libzstd decodes them to or raise. Containers laid out
the way the reference's encoder writes them (norm weights as lowcard, integer
buffers as zstd, matrices in the reference's rANS formats) load bit-exactly.
"""
from __future__ import annotations

import hashlib
import sys

import numpy as np
import pytest
import torch

import oracle
from oracle import zstd_lib

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not zstd_lib.available(), reason="libzstd is not installed")]

LEVELS = [-5, 1, 3, 9, 19, 22]


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _datasets() -> dict[str, bytes]:
    rng = np.random.default_rng(0)
    d = {}
    for n in (1, 7, 100, 4096, 200_000):
        d[f"random{n}"] = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        d[f"zeros{n}"] = bytes(n)
    for n in (4096, 14336, 1_000_000):               # norm-weight indices: 16 values, skewed
        d[f"lowcard{n}"] = np.clip(np.rint(rng.normal(0, 3, n)) + 8, 0, 15).astype(np.uint8).tobytes()
    x = (rng.standard_normal(300_000) * 0.02).astype(np.float32).view(np.uint32).astype(np.uint64)
    d["bf16"] = ((x + 0x7FFF + ((x >> 16) & 1)) >> 16).astype(np.uint16).tobytes()
    d["arange_i64"] = np.arange(100_000, dtype=np.int64).tobytes()
    words = np.array([b"alpha ", b"beta ", b"gamma ", b"delta ", b"epsilon ", b"zeta ", b"eta\n", b"theta, "])
    text = bytearray(b"".join(words[rng.integers(0, 8, 90_000)]))
    for _ in range(60):                              # long-range repeats
        a = int(rng.integers(0, len(text) - 5000))
        text += text[a:a + int(rng.integers(100, 5000))]
    d["text"] = bytes(text)
    return d


def _decode_batch(frames: list[bytes], sizes: list[int]):
    """One bs_zstd_decode launch over all frames; returns (outputs, per-task
    decoded length, status word value)."""
    from bigsmall_amd.codecs.zstd_gpu import ZstdLaunch
    from bigsmall_amd.device import StatusWord
    dev = torch.device("cuda", 0)
    src_off = np.cumsum([0] + [len(f) for f in frames])
    dst_off = np.cumsum([0] + list(sizes))
    src = torch.from_numpy(np.frombuffer(b"".join(frames) + b"\0", np.uint8).copy()).to(dev)
    dst = torch.zeros(int(dst_off[-1]) + 1, dtype=torch.uint8, device=dev)
    z = ZstdLaunch(dev)
    for i, f in enumerate(frames):
        z.add_frame(src.data_ptr() + int(src_off[i]), len(f), dst.data_ptr() + int(dst_off[i]), sizes[i])
    st = StatusWord(dev)
    z.launch(st)
    torch.cuda.synchronize()
    host = dst.cpu().numpy()
    outs = [host[dst_off[i]:dst_off[i + 1]].tobytes() for i in range(len(frames))]
    return outs, z.out_len.cpu().tolist(), int(st.t.item())


def test_frames_every_level_in_one_launch():
    data = _datasets()
    frames, sizes, names = [], [], []
    for name, raw in data.items():
        for lv in LEVELS:
            frames.append(zstd_lib.compress(raw, lv))
            sizes.append(len(raw))
            names.append(f"{name} L{lv}")
    t = data["text"]
    for extra, f in (("checksum", zstd_lib.compress(t, 3, checksum=True)),
                     ("no content size", zstd_lib.compress(t, 19, content_size=False))):
        frames.append(f)
        sizes.append(len(t))
        names.append(f"text {extra}")
    _say(f"[zstd] {len(frames)} frames, {sum(sizes)} bytes, one launch")
    outs, lens, status = _decode_batch(frames, sizes)
    assert status == 0, hex(status)
    for name, f, n, got, ln in zip(names, frames, sizes, outs, lens):
        assert ln == n, name
        assert got == zstd_lib.decompress(f, n), name


@pytest.mark.parametrize("name", sorted(zstd_lib.KNOWN_FRAMES))
def test_hand_built_frames(name):
    frame, want = zstd_lib.KNOWN_FRAMES[name]
    _say(f"[zstd] hand-built frame {name}")
    outs, lens, status = _decode_batch([frame], [len(want)])
    assert status == 0 and lens == [len(want)] and outs[0] == want


def test_back_to_back_frames_and_multiblock():
    rng = np.random.default_rng(1)
    big = bytearray(np.clip(np.rint(rng.normal(0, 9, 6_000_000)) + 128, 0, 255).astype(np.uint8).tobytes())
    big[3_000_000:3_400_000] = big[100_000:500_000]  # a repeat 2.9 MB back, across many blocks
    big = bytes(big)
    small = b"back to back " * 100
    frame = zstd_lib.compress(small, 3) + b"\x50\x2a\x4d\x18\x02\x00\x00\x00ab" + zstd_lib.compress(big, 19)
    _say("[zstd] 6 MB level 19 after a small frame and a skippable frame")
    outs, lens, status = _decode_batch([frame, zstd_lib.compress(big, 1)], [len(small) + len(big), len(big)])
    assert status == 0, hex(status)
    assert outs[0] == small + big and outs[1] == big


def test_wrong_size_is_reported():
    from bigsmall_amd import _native
    f = zstd_lib.compress(b"abc" * 1000, 3)
    _say("[zstd] size mismatch")
    _, lens, status = _decode_batch([f, f], [2999, 3001])
    assert lens == [0, 0] and status & _native.BS_DEV_ERR_COUNT


def test_corrupted_frames_decode_like_libzstd_or_fail():
    rng = np.random.default_rng(2)
    data = _datasets()
    frames, sizes, want = [], [], []
    for name in ("lowcard4096", "text", "bf16", "random4096"):
        raw = data[name]
        for lv in (1, 19):
            f = zstd_lib.compress(raw, lv)
            for k in range(40):
                g = bytearray(f)
                if k % 3 == 2:
                    g = g[:int(rng.integers(0, len(g)))]
                else:
                    g[int(rng.integers(0, len(g)))] ^= 1 << int(rng.integers(0, 8))
                g = bytes(g) or b"\0"
                frames.append(g)
                sizes.append(len(raw))
                try:
                    want.append(zstd_lib.decompress(g, len(raw)))
                except ValueError:
                    want.append(None)
    _say(f"[zstd] {len(frames)} corrupted frames, one launch")
    outs, lens, status = _decode_batch(frames, sizes)
    decoded = 0
    for i, (got, ln, w) in enumerate(zip(outs, lens, want)):
        if ln == sizes[i]:
            decoded += 1
            assert w is not None and got == w, i            # decoded only where libzstd agrees, to its bytes
        else:
            assert ln == 0, i
    assert status != 0 and 0 < decoded < len(frames)


def _bf16_words(rng, n, mean=0.0, std=0.02):
    x = (mean + rng.standard_normal(n) * std).astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((x + 0x7FFF + ((x >> 16) & 1)) >> 16).astype(np.uint16)


def _reference_layout_container(path):
    """A 2-layer model laid out the way the reference's encoder writes it with
    forced rANS-family codecs: matrices as bf16_parallel_v1 / bf16_se_tans,
    RMSNorm weights (1 + N(0, 0.01), about 16 distinct bf16 values) as
    special/lowcard, integer and fp32 buffers as zstd (level 9), a causal mask
    as a 1-byte lowcard, a tiny tensor raw and lm_head tied to the embedding
    (bigsmall/encoder.py:57, 386-470; codec_registry.py:183-188)."""
    from bigsmall_amd import container
    rng = np.random.default_rng(4)
    items = []
    for i in range(2):
        p = f"model.layers.{i}."
        items.append((p + "self_attn.q_proj.weight", [256, 512], "bfloat16", _bf16_words(rng, 256 * 512), "par"))
        items.append((p + "mlp.down_proj.weight", [512, 256], "bfloat16", _bf16_words(rng, 512 * 256), "tans"))
        for norm in ("input_layernorm.weight", "post_attention_layernorm.weight"):
            items.append((p + norm, [4096], "bfloat16", _bf16_words(rng, 4096, 1.0, 0.01), "lowcard"))
        items.append((p + "attn.bias", [64, 64], "bool", np.tril(np.ones((64, 64), np.uint8)).reshape(-1), "lowcard"))
    items.append(("model.embed_tokens.weight", [1000, 256], "bfloat16", _bf16_words(rng, 256_000), "par"))
    items.append(("model.norm.weight", [4096], "bfloat16", _bf16_words(rng, 4096, 1.0, 0.01), "lowcard"))
    items.append(("position_ids", [1, 8192], "int64", np.arange(8192, dtype=np.int64), "zstd"))
    items.append(("rotary.inv_freq", [64], "float32",
                  (1.0 / 10000 ** (np.arange(0, 128, 2) / 128)).astype(np.float32), "zstd"))
    items.append(("model.layers.0.self_attn.q_proj.bias", [16], "bfloat16", np.zeros(16, np.uint16), "raw"))
    data, tensors, src = bytearray(), [], {}
    for name, shape, dtype, arr, how in items:
        raw = arr.tobytes()
        src[name] = raw
        extra = None
        if how == "par":
            codec, blob = "bf16_parallel_v1", oracle.par1_encode(arr)
        elif how == "tans":
            codec, blob = "bf16_se_tans", oracle.tans_encode(arr)
        elif how == "lowcard":
            codec, (blob, extra) = "special", zstd_lib.encode_lowcard(raw, arr.itemsize)
            extra = dict(extra, special_kind="lowcard")
        elif how == "zstd":
            codec, (blob, extra) = "zstd", zstd_lib.encode_zstd(raw)
        else:
            codec, blob = "raw", raw
        tensors.append({"name": name, "shape": shape, "dtype": dtype, "codec": codec,
                        "special": "lowcard" if how == "lowcard" else None, "compressed_bytes": len(blob),
                        "offset": len(data), "md5": hashlib.md5(raw).hexdigest(), "extra": extra})
        data += blob
    emb = next(t for t in tensors if t["name"] == "model.embed_tokens.weight")
    tensors.append({"name": "lm_head.weight", "shape": emb["shape"], "dtype": "bfloat16", "codec": "tied_ref",
                    "special": None, "compressed_bytes": 0, "offset": 0, "md5": emb["md5"],
                    "extra": {"tied_to": "model.embed_tokens.weight"}})
    src["lm_head.weight"] = src["model.embed_tokens.weight"]
    header = {"format": "bf16", "mode": "balanced", "model_type": "llm", "base_model": None,
              "tensor_count": len(tensors), "tensors": tensors}
    container.write_container(path, header, bytes(data), format_version=2)
    return src


def _host_bytes(t: torch.Tensor) -> bytes:
    return t.detach().contiguous().cpu().view(-1).view(torch.uint8).numpy().tobytes()


def test_reference_layout_container_loads(tmp_path):
    from bigsmall_amd import container, decoder
    from bigsmall_amd.streaming import StreamingLoader
    from bigsmall_amd.verify import verify
    p = tmp_path / "ref_layout.bs"
    src = _reference_layout_container(p)
    _say("[zstd] reference-layout container: load")
    out = decoder.load(p, device="cuda")
    assert set(out) == set(src)
    for k, raw in src.items():
        assert out[k].is_cuda and _host_bytes(out[k]) == raw, k
    _say("[zstd] decompress / verify / _decode_blob")
    host = decoder.decompress(p)
    header, off = container.read_header(p)
    for i, t in enumerate(header["tensors"]):
        assert hashlib.md5(host[t["name"]].tobytes()).hexdigest() == t["md5"], t["name"]
        raw = decoder._decode_blob(t, container.read_blob(p, header, off, i))
        assert raw is None if t["codec"] == "tied_ref" else raw == src[t["name"]], t["name"]
    assert verify(p)
    _say("[zstd] streaming")
    with StreamingLoader(p, prefetch=1) as L:
        for li, layer in L.iter_layers():
            for k, t in layer.items():
                assert _host_bytes(t) == src[k], k
        nl = L.load_non_layer_tensors()
        assert all(_host_bytes(v) == src[k] for k, v in nl.items())


def test_lowcard_index_past_table_raises():
    from bigsmall_amd.codecs.zstd_gpu import decode_lowcard
    from bigsmall_amd.exceptions import DecodeError
    raw = np.arange(16, dtype=np.uint16).repeat(64).tobytes()
    blob = bytearray(zstd_lib.encode_lowcard(raw, 2)[0])
    blob[1] = 15                                     # table cut to 15 values; index 15 now points past it
    blob = blob[:2 + 15 * 2] + blob[2 + 16 * 2:]
    _say("[zstd] lowcard index past its table")
    assert decode_lowcard(zstd_lib.encode_lowcard(raw, 2)[0], {}, len(raw)) == raw
    with pytest.raises(DecodeError):
        decode_lowcard(bytes(blob), {}, len(raw))


def test_plugin_api_decoders():
    from bigsmall_amd.codecs.zstd_gpu import decode_special, decode_zstd
    raw = np.arange(5000, dtype=np.int64).tobytes()
    blob, extras = zstd_lib.encode_zstd(raw)
    _say("[zstd] plugin decoders")
    assert decode_zstd(blob, extras) == raw                 # size from the frame header
    from bigsmall_amd import codec_registry
    assert codec_registry.get_codec("zstd")[1](blob, extras, 5000) == raw
    assert decode_zstd(blob, extras, len(raw)) == raw
    norm = _bf16_words(np.random.default_rng(5), 4096, 1.0, 0.01).tobytes()
    lb, le = zstd_lib.encode_lowcard(norm, 2)
    assert decode_special(lb, dict(le, special_kind="lowcard"), len(norm)) == norm
    with pytest.raises(ValueError):
        decode_special(lb, {"special_kind": "wpe_delta"}, len(norm))


def _write_delta_container(path, base: dict, ft: dict, extra_ft: dict):
    """A delta container as bigsmall/encoder.py:705-824 writes it: tensors that
    match the base in shape, dtype and size as zstd_xor_delta (level 19, extras
    is_xor_delta), a tensor with no base entry standalone (here raw bytes as
    zstd, the reference's route for fmt "raw")."""
    from bigsmall_amd import container
    data, tensors = bytearray(), []
    for name, arr in list(ft.items()) + list(extra_ft.items()):
        raw = arr.tobytes()
        if name in base:
            blob, extra = zstd_lib.encode_zstd(np.frombuffer(raw, np.uint8) ^ np.frombuffer(base[name].tobytes(),
                                                                                          np.uint8), 19)
            codec, extra, special = "zstd_xor_delta", dict(extra, is_xor_delta=True), "delta"
        else:
            (blob, extra), codec, special = zstd_lib.encode_zstd(raw), "zstd", None
        tensors.append({"name": name, "shape": list(arr.shape), "dtype": "bfloat16" if arr.dtype == np.uint16
                        else "int64", "codec": codec, "special": special, "compressed_bytes": len(blob),
                        "offset": len(data), "md5": hashlib.md5(raw).hexdigest(), "extra": extra})
        data += blob
    header = {"format": "bf16", "mode": "balanced", "model_type": "delta", "base_model": "base",
              "tensor_count": len(tensors), "tensors": tensors}
    container.write_container(path, header, bytes(data))


def test_delta_roundtrip_against_safetensors_and_bs_base(tmp_path):
    """Mirror of the reference's tests/test_delta.py:13-53: a fine-tune that
    differs from its base in ~1% of the elements, stored as a delta, comes
    back md5-identical from decompress_delta with the base given as
    safetensors or as a .bs container."""
    from safetensors.torch import save_file

    import bigsmall_amd as bs
    from bigsmall_amd import container
    rng = np.random.default_rng(8)
    shapes = {"embed.weight": (2000, 256), "layer.0.weight": (256, 512), "layer.1.weight": (512, 256)}
    base = {k: _bf16_words(rng, int(np.prod(s)), 0.0, 1.0).reshape(s) for k, s in shapes.items()}
    ft = {}
    for k, v in base.items():                    # v + 0.01 where a 1% mask is set, rounded to bf16
        f = (v.astype(np.uint32) << 16).view(np.float32)
        m = rng.random(v.shape) < 0.01
        x = (f + np.float32(0.01) * m).astype(np.float32).view(np.uint32).astype(np.uint64)
        ft[k] = ((x + 0x7FFF + ((x >> 16) & 1)) >> 16).astype(np.uint16)
    extra = {"position_ids": np.arange(512, dtype=np.int64).reshape(1, 512)}
    delta = tmp_path / "delta.bs"
    _write_delta_container(delta, base, ft, extra)
    base_st = tmp_path / "base.safetensors"
    save_file({k: torch.from_numpy(v.view(np.int16)).view(torch.bfloat16) for k, v in base.items()}, str(base_st))
    base_bs = tmp_path / "base.bs"
    bs.compress(base_st, base_bs)
    header, _ = container.read_header(delta)
    for base_src in (base_st, base_bs):
        _say(f"[zstd] decompress_delta against {base_src.suffix}")
        out = bs.decompress_delta(delta, base_src)
        for t in header["tensors"]:
            assert hashlib.md5(out[t["name"]].tobytes()).hexdigest() == t["md5"], t["name"]
        dev = bs.load_delta(delta, base_src)
        assert all(dev[k].is_cuda for k in dev)
        assert _host_bytes(dev["layer.0.weight"]) == ft["layer.0.weight"].tobytes()
    _say("[zstd] delta bytes without a base")
    from bigsmall_amd import decoder
    plain = decoder.load(delta)                  # no base: the XOR delta itself, as _decode_blob returns it
    want = (np.frombuffer(ft["layer.1.weight"].tobytes(), np.uint8) ^
            np.frombuffer(base["layer.1.weight"].tobytes(), np.uint8)).tobytes()
    assert _host_bytes(plain["layer.1.weight"]) == want
