"""Property-based GPU round trips (hypothesis), after the reference's
tests/test_property_based.py: any 1-3-D tensor of bf16 / fp16 / fp32 / fp8
compresses and loads back bit-exactly through the GPU decode, `verify`
passes; the GPU encoder's blob equals the host encoder's for any size.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

hyp = pytest.importorskip("hypothesis")
from hypothesis import HealthCheck, given, settings, strategies as st  # noqa: E402

pytestmark = pytest.mark.gpu
SETTINGS = dict(max_examples=15, deadline=None,
                suppress_health_check=[HealthCheck.too_slow, HealthCheck.function_scoped_fixture])


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@given(shape=st.lists(st.integers(1, 64), min_size=1, max_size=3),
       dtype=st.sampled_from(["bfloat16", "float16", "float32", "float8_e4m3fn"]), seed=st.integers(0, 2**31),
       scale=st.sampled_from([1e-3, 0.02, 1.0, 300.0]))
@settings(**SETTINGS)
def test_property_compress_load_roundtrip(tmp_path_factory, shape, dtype, seed, scale):
    from bigsmall_amd.decoder import load
    from bigsmall_amd.encoder import compress
    from bigsmall_amd.verify import verify
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    t = x.to(getattr(torch, dtype))
    p = tmp_path_factory.mktemp("prop") / "t.bs"
    compress({"model.layers.0.mlp.up_proj.weight": t, "model.norm.weight": t.flatten()[:7].clone()}, p)
    _say(f"[prop] {dtype} {shape} scale={scale}")
    out = load(p, device="cuda")
    for k, ref in (("model.layers.0.mlp.up_proj.weight", t), ("model.norm.weight", t.flatten()[:7])):
        got = out[k].cpu()
        assert got.dtype == ref.dtype and tuple(got.shape) == tuple(ref.shape)
        assert got.contiguous().view(torch.uint8).numpy().tobytes() == \
            ref.contiguous().view(torch.uint8).numpy().tobytes(), k
    assert verify(p)


@given(n=st.integers(1, 300_000), seed=st.integers(0, 2**31), steps=st.sampled_from([16, 64, 256, 448]))
@settings(**SETTINGS)
def test_property_gpu_encoder_matches_host(n, seed, steps):
    from bigsmall_amd.codecs import bf16_chunked as bc
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * 10.0 ** rng.uniform(-3, 1)).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    w = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    t = torch.from_numpy(w.view(np.int16).copy()).view(torch.bfloat16).cuda()
    arena, [(off, ln)] = bc.encode_device([t], steps=steps)
    assert arena[off:off + ln].cpu().numpy().tobytes() == bc.encode_array(w, steps=steps, mode=bc.MODE_DENSE,
                                                                            lanes=128)
