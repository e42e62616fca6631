"""GPU mirrors of the reference's codec tests for the formats this engine
decodes from the reference's encoders (tests/test_tans.py:15-37,
tests/test_single_kernel.py:15-40, tests/test_gpu_kernel.py:38-80). The
reference encodes with its own codec and decodes it back; here the blob is
written by the oracle's encoder (byte-identical to the reference's, pinned by
the golden fixtures) and decoded through this engine's plugin entry points on
the GPU. Bar: bit-exact (md5 of the raw bytes)."""
from __future__ import annotations

import hashlib
import os
import struct

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

SPECIALS = [0x7FC0, 0x7F80, 0xFF80, 0x0000, 0x8000, 0x0001, 0x0080, 0x3F80]


def _md5(b: bytes) -> str:
    return hashlib.md5(b).hexdigest()


def _gauss_raw(seed: int, n: int) -> bytes:
    torch.manual_seed(seed)
    return (torch.randn(n) * 0.02).to(torch.bfloat16).view(torch.uint8).numpy().tobytes()


def _edge_raw() -> bytes:
    torch.manual_seed(1)
    normals = (torch.randn(4096) * 0.02).to(torch.bfloat16).view(torch.uint8).numpy()
    return b"".join(struct.pack("<H", w) for w in SPECIALS) + normals.tobytes()


@pytest.fixture(scope="module", autouse=True)
def _built():
    oracle.build()


@pytest.mark.parametrize("n", [256, 65536, 1 << 18])
def test_tans_roundtrip_gaussian(n):
    from bigsmall_amd.codecs import bf16_tans
    raw = _gauss_raw(0, n)
    blob = oracle.tans_encode(np.frombuffer(raw, np.uint16))
    assert _md5(bf16_tans.decode(blob, {}, n)) == _md5(raw)


def test_tans_roundtrip_edge_cases():
    from bigsmall_amd.codecs import bf16_tans
    raw = _edge_raw()
    blob = oracle.tans_encode(np.frombuffer(raw, np.uint16))
    assert bf16_tans.decode(blob, {}, len(raw) // 2) == raw


@pytest.mark.parametrize("n", [4096, 65536, 1 << 18])
def test_single_kernel_roundtrip_gaussian(n):
    from bigsmall_amd.codecs import single_kernel
    raw = _gauss_raw(0, n)
    blob = oracle.sk_encode(np.frombuffer(raw, np.uint16))
    assert _md5(single_kernel.decode(blob, {}, n)) == _md5(raw)


def test_single_kernel_roundtrip_edge_cases():
    from bigsmall_amd.codecs import single_kernel
    raw = _edge_raw()
    blob = oracle.sk_encode(np.frombuffer(raw, np.uint16))
    assert single_kernel.decode(blob, {}, len(raw) // 2) == raw


def test_gpu_decode_lossless():
    """tests/test_gpu_kernel.py:38-52: 64 streams, 256K elements; the GPU
    output equals the CPU decoder's (the oracle's restatement) and the source."""
    from bigsmall_amd import kernels
    n = 1 << 18
    raw = _gauss_raw(0, n)
    blob = oracle.par1_encode(np.frombuffer(raw, np.uint16), n_streams=64)
    cpu = oracle.par1_decode(blob, n)
    gpu = kernels.decode_bf16_parallel(blob, {}, n)
    assert _md5(cpu) == _md5(raw) and _md5(gpu) == _md5(raw) and cpu == gpu


def test_kernels_module_picks_gpu_backend():
    from bigsmall_amd import kernels
    kernels._GPU_BACKEND = None
    os.environ.pop("BIGSMALL_FORCE_CPU", None)
    assert kernels.use_gpu() is True and kernels.backend_name() == "hip"


def test_force_cpu_env_disables_gpu():
    """tests/test_gpu_kernel.py:67-80. The reference then decodes on its CPU
    path; this engine has none, so decoding raises instead."""
    from bigsmall_amd import kernels
    kernels._GPU_BACKEND = None
    os.environ["BIGSMALL_FORCE_CPU"] = "1"
    try:
        assert kernels.use_gpu() is False and kernels.backend_name() == "cpu"
        blob = oracle.par1_encode(np.frombuffer(_gauss_raw(0, 1024), np.uint16))
        with pytest.raises(RuntimeError):
            kernels.decode_bf16_parallel(blob, {}, 1024)
    finally:
        del os.environ["BIGSMALL_FORCE_CPU"]
        kernels._GPU_BACKEND = None
