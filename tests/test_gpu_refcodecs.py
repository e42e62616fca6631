"""GPU parity of the reference's rANS-family formats (bf16_parallel_v1,
bf16_se_tans, bf16_se_single_kernel) decoded by bs_refcodec_decode.

Bar: bit-exact. Inputs are (1) the golden blobs written by the reference's own
encoders (tests/golden/ref_vectors.npz) and (2) larger blobs from the oracle's
encoders, which are byte-identical to the reference's on every golden vector
(tests/test_oracle_golden.py). Each GPU output must equal the source words and
the oracle's CPU decode of the same blob.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

CODECS = {
    "bf16_parallel_v1": (oracle.par1_encode, oracle.par1_decode, "par1_"),
    "bf16_se_tans": (oracle.tans_encode, oracle.tans_decode, "tans_"),
    "bf16_se_single_kernel": (oracle.sk_encode, oracle.sk_decode, "sk_"),
}


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _bf16(x: np.ndarray) -> np.ndarray:
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.fixture(scope="module")
def gpu():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    oracle.build()
    return torch


def _decode(codec, blob, n):
    from bigsmall_amd.codecs import _refstreams
    return _refstreams.decode_host(codec, blob, n)


@pytest.mark.parametrize("codec", list(CODECS))
def test_reference_golden_blobs(gpu, golden, codec):
    prefix = CODECS[codec][2]
    seen = 0
    for k in sorted(golden):
        if not k.startswith(prefix):
            continue
        name = k[len(prefix):].rsplit("_N", 1)[0] if prefix == "par1_" else k[len(prefix):]
        words = golden[f"in_{name}"].astype("<u2")
        _say(f"[ref] {codec} golden {k} n={words.size}")
        assert _decode(codec, golden[k].tobytes(), words.size) == words.tobytes(), k
        seen += 1
    assert seen >= 7


@pytest.mark.parametrize("codec", list(CODECS))
@pytest.mark.parametrize("kind", ["gauss", "studentt", "halfzero", "uniform"])
def test_oracle_encoded_larger(gpu, codec, kind):
    enc, dec, _ = CODECS[codec]
    rng = np.random.default_rng(len(kind))
    n = 300_007 if codec != "bf16_parallel_v1" else 1_000_003
    if kind == "gauss":
        w = _bf16(rng.standard_normal(n) * 0.02)
    elif kind == "studentt":
        w = _bf16(rng.standard_t(3, n) * 0.02 / np.sqrt(3))
    elif kind == "halfzero":
        w = _bf16(rng.standard_normal(n) * 0.02)
        w[rng.permutation(n)[: n // 2]] = 0
    else:
        w = rng.integers(0, 65536, n).astype(np.uint16)
    blob = enc(w)
    _say(f"[ref] {codec} {kind} n={n} blob={len(blob)}")
    got = _decode(codec, blob, n)
    assert got == w.tobytes()
    assert got == dec(blob, n)


def test_parallel_stream_counts(gpu):
    rng = np.random.default_rng(5)
    w = _bf16(rng.standard_normal(70_001) * 0.02)
    for ns in [1, 3, 64, 128, 257, 1024]:
        blob = oracle.par1_encode(w, ns)
        _say(f"[ref] bf16_parallel_v1 N={ns}")
        assert _decode("bf16_parallel_v1", blob, w.size) == w.tobytes()


def test_corrupt_stream_is_reported(gpu):
    from bigsmall_amd.exceptions import DecodeError
    rng = np.random.default_rng(6)
    w = _bf16(rng.standard_normal(50_000) * 0.02)
    blob2 = bytearray(oracle.tans_encode(w))
    # flip a byte deep inside the SE renorm words: the stream no longer ends in state L
    se_n = int.from_bytes(blob2[4:6], "little")
    se_cw = 4 + 2 + 6 * se_n + 4
    blob2[se_cw + 200] ^= 0x5A
    _say("[ref] corrupt tans stream -> DecodeError")
    with pytest.raises((DecodeError, ValueError)):
        _decode("bf16_se_tans", bytes(blob2), w.size)


@pytest.mark.parametrize("codec", list(CODECS))
@pytest.mark.parametrize("n", [30_000, 80_000])
def test_single_byte_corruptions_decode_or_raise(gpu, codec, n):
    """Single-byte corruptions of a reference-format blob (half in its first
    4 KB of framing and tables, half anywhere) either decode or raise
    ValueError / DecodeError, on the one-lane path (below 65,536 elements) and
    on the wave-serial path; the clean blob still decodes afterwards."""
    from bigsmall_amd.exceptions import DecodeError
    rng = np.random.default_rng(n + len(codec))
    w = _bf16(rng.standard_normal(n) * 0.02)
    blob = CODECS[codec][0](w)
    _say(f"[ref] {codec} n={n}: 60 single-byte corruptions")
    outcomes = {"ok": 0, "raised": 0}
    for t in range(60):
        bad = bytearray(blob)
        pos = int(rng.integers(0, min(len(blob), 4096))) if t % 2 else int(rng.integers(0, len(blob)))
        bad[pos] ^= int(rng.integers(1, 256))
        try:
            _decode(codec, bytes(bad), n)
            outcomes["ok"] += 1
        except (ValueError, DecodeError):
            outcomes["raised"] += 1
    _say(f"[ref] outcomes {outcomes}")
    assert _decode(codec, blob, n) == w.tobytes()
    assert outcomes["raised"] > 0, outcomes


def test_serial_batch_mixed_formats(gpu):
    """One bs_refcodec_decode_serial_batch launch decodes tensors of all three
    formats side by side (different sizes, stream counts and exponent sets);
    each output equals its source words, and equals the one-tensor entry
    point's output for the same blob."""
    from bigsmall_amd.codecs import _refstreams
    from bigsmall_amd.device import StatusWord, upload_bytes
    torch = gpu
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(21)
    srcs = [("bf16_parallel_v1", _bf16(rng.standard_normal(300_001) * 0.02)),
            ("bf16_se_tans", _bf16(rng.standard_t(3, 200_003) * 0.02)),
            ("bf16_se_single_kernel", _bf16(rng.standard_normal(131_072) * 0.5)),
            ("bf16_parallel_v1", _bf16(rng.standard_normal(70_000) * 0.02)),
            ("bf16_se_tans", rng.integers(0, 65536, 90_000).astype(np.uint16))]
    blobs = [CODECS[c][0](w) for c, w in srcs]
    d_blobs = [upload_bytes(b, dev) for b in blobs]
    outs = [torch.empty(w.size, dtype=torch.int16, device=dev) for _, w in srcs]
    items = [(_refstreams.PARSERS[c](b, w.size), d.data_ptr(), o.data_ptr())
             for (c, w), b, d, o in zip(srcs, blobs, d_blobs, outs)]
    assert all(_refstreams.serial_ok(p) for p, _, _ in items)
    st = StatusWord(dev)
    batch = _refstreams.RefBatch(items, dev)
    _say(f"[ref] serial batch of {len(items)} tensors, totals {batch.totals}")
    for rep in range(2):                 # the second launch reuses the scratch of the first
        batch.launch(st.ptr, torch.cuda.current_stream(dev).cuda_stream)
        torch.cuda.synchronize()
        st.check("serial batch")
        for (c, w), o in zip(srcs, outs):
            assert o.cpu().numpy().view(np.uint16).tobytes() == w.tobytes(), (rep, c, w.size)
    for (c, w), b in zip(srcs, blobs):
        assert _decode(c, b, w.size) == w.tobytes(), c


def test_serial_batch_with_shared_xcd_bins(gpu):
    """Twelve tensors in one batch: more than the eight XCD bins, so bins hold
    several tensors and only the first of each reads its SE table through the
    scalar cache (the others from LDS). The layout obeys the bins (every
    task's SE groups inside one bin, the task array ascending, the grid 8C
    groups) and every output equals its source."""
    from bigsmall_amd.codecs import _refstreams
    from bigsmall_amd.device import StatusWord, upload_bytes
    torch = gpu
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(23)
    kinds = ["bf16_parallel_v1", "bf16_se_tans", "bf16_se_single_kernel"]
    srcs = [(kinds[i % 3], _bf16(rng.standard_normal(int(rng.integers(70_000, 260_000))) * 0.02))
            for i in range(12)]
    blobs = [CODECS[c][0](w) for c, w in srcs]
    d_blobs = [upload_bytes(b, dev) for b in blobs]
    outs = [torch.empty(w.size, dtype=torch.int16, device=dev) for _, w in srcs]
    items = [(_refstreams.PARSERS[c](b, w.size), d.data_ptr(), o.data_ptr())
             for (c, w), b, d, o in zip(srcs, blobs, d_blobs, outs)]
    batch = _refstreams.RefBatch(items, dev)
    off = batch.p_tasks - batch.dev.data_ptr()
    n = len(items)
    tasks = batch.dev[off:off + n * _refstreams.REF_TASK_DTYPE.itemsize].cpu().numpy().view(_refstreams.REF_TASK_DTYPE)
    C = batch.totals[0] // _refstreams.XCD_BINS
    per = 4
    begins = tasks["se_group_begin"].astype(np.int64)
    assert batch.totals[0] == _refstreams.XCD_BINS * C and np.all(np.diff(begins) > 0)
    for t in tasks:
        g = -(-int(t["n_streams"]) // per)
        assert int(t["se_group_begin"]) // C == (int(t["se_group_begin"]) + g - 1) // C
    bins = begins // C
    scalar = (tasks["flags"] & _refstreams.FLAG_SE_SCALAR) != 0
    assert len(set(bins.tolist())) == _refstreams.XCD_BINS      # every bin used
    assert all(scalar[bins == b].sum() <= 1 for b in set(bins.tolist()))
    st = StatusWord(dev)
    _say(f"[ref] serial batch of {n} tensors in shared bins, totals {batch.totals}, scalar {int(scalar.sum())}")
    batch.launch(st.ptr, torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    st.check("serial batch, shared bins")
    for (c, w), o in zip(srcs, outs):
        assert o.cpu().numpy().view(np.uint16).tobytes() == w.tobytes(), (c, w.size)


def test_serial_batch_rejects_inconsistent_task(gpu):
    """A task whose scratch lies outside the work buffer, or whose element
    count is zero, is reported (BS_DEV_ERR_HEADER) and skipped by every kernel
    of the batch; the other tasks still decode."""
    from bigsmall_amd.codecs import _refstreams
    from bigsmall_amd.device import StatusWord, upload_bytes
    from bigsmall_amd.exceptions import DecodeError
    torch = gpu
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(22)
    srcs = [_bf16(rng.standard_normal(100_000) * 0.02), _bf16(rng.standard_normal(80_000) * 0.02)]
    blobs = [oracle.tans_encode(w) for w in srcs]
    d_blobs = [upload_bytes(b, dev) for b in blobs]
    for field, value in (("work_offset", 1 << 40), ("n_out", 0), ("work_offset", 128)):
        outs = [torch.zeros(w.size, dtype=torch.int16, device=dev) for w in srcs]
        items = [(_refstreams.PARSERS["bf16_se_tans"](b, w.size), d.data_ptr(), o.data_ptr())
                 for w, b, d, o in zip(srcs, blobs, d_blobs, outs)]
        batch = _refstreams.RefBatch(items, dev)
        off = batch.p_tasks - batch.dev.data_ptr()
        tasks = batch.dev[off:off + 2 * _refstreams.REF_TASK_DTYPE.itemsize].cpu().numpy().view(_refstreams.REF_TASK_DTYPE).copy()
        # the batch orders its task array by its grid layout: find the second tensor's task by its output
        (j,) = np.flatnonzero(tasks["out"] == outs[1].data_ptr())
        tasks[field][j] = value
        batch.dev[off:off + tasks.nbytes].copy_(torch.from_numpy(tasks.view(np.uint8)))
        st = StatusWord(dev)
        _say(f"[ref] serial batch with task 1 {field}={value}")
        batch.launch(st.ptr, torch.cuda.current_stream(dev).cuda_stream)
        torch.cuda.synchronize()
        with pytest.raises(DecodeError):
            st.check("serial batch")
        assert outs[0].cpu().numpy().view(np.uint16).tobytes() == srcs[0].tobytes()
