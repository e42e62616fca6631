"""The entry point that allocates nothing: bs_zstd_decode_static (the zstd
decode with its literal slices in a static device array) against the same
tasks decoded by bs_zstd_decode with a caller-allocated work buffer.

Bar: bit-exact. Two calls in a row, the second with fewer and smaller frames,
so the second runs over scratch the first left behind; both must equal the
work-buffer entry point's output and the frames' source bytes. Then two calls
on two streams issued back to back, which the library orders on the shared
array: each must decode its own frames exactly. More tasks than the static
array holds are refused on the host, before any launch.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import zstd_lib

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not zstd_lib.available(), reason="libzstd is not installed")]


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _frames(seed: int, count: int, max_n: int):
    rng = np.random.default_rng(seed)
    srcs, frames = [], []
    for i in range(count):
        n = int(rng.integers(1, max_n))
        if i % 3 == 0:
            src = np.clip(np.rint(rng.normal(0, 3, n)) + 8, 0, 15).astype(np.uint8).tobytes()
        elif i % 3 == 1:
            src = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        else:
            src = (b"static scratch " * (n // 15 + 1))[:n]
        srcs.append(src)
        frames.append(zstd_lib.compress(src, [1, 3, 19][i % 3]))
    return srcs, frames


def _prepare(srcs, frames):
    """Device copies of the frames, output buffers, the task table and the
    status word, all in place (synchronised) before any decode is issued."""
    from bigsmall_amd.codecs.zstd_gpu import ZSTD_TASK_DTYPE
    from bigsmall_amd.device import StatusWord, upload_bytes
    dev = torch.device("cuda", 0)
    d_src = [upload_bytes(np.frombuffer(f, np.uint8), dev) for f in frames]
    d_dst = [torch.full((len(s),), 0xA5, dtype=torch.uint8, device=dev) for s in srcs]
    t = np.zeros(len(frames), ZSTD_TASK_DTYPE)
    for i, (a, b, f) in enumerate(zip(d_src, d_dst, frames)):
        t[i] = (a.data_ptr(), len(f), b.data_ptr(), b.numel(), 0)
    d_tasks = upload_bytes(t.view(np.uint8), dev)
    out_len = torch.zeros(len(frames), dtype=torch.int64, device=dev)
    st = StatusWord(dev)
    torch.cuda.synchronize(dev)
    return d_src, d_dst, d_tasks, out_len, st


def _issue(prep, static: bool, stream=None):
    """Issue one decode call over prepared buffers on `stream` (the current
    stream by default) without waiting for it; returns what _collect needs,
    which keeps every buffer alive until then."""
    from bigsmall_amd import _native
    d_src, d_dst, d_tasks, out_len, st = prep
    dev = torch.device("cuda", 0)
    L = _native.lib()
    frames = len(d_src)
    s = (stream or torch.cuda.current_stream(dev)).cuda_stream
    work = None
    if static:
        rc = L.bs_zstd_decode_static(d_tasks.data_ptr(), frames, out_len.data_ptr(), st.ptr, s)
        _native.check(rc, "bs_zstd_decode_static")
    else:
        wb = int(L.bs_zstd_work_bytes(frames))
        work = torch.empty(wb, dtype=torch.uint8, device=dev)
        rc = L.bs_zstd_decode(d_tasks.data_ptr(), frames, work.data_ptr(), wb, out_len.data_ptr(), st.ptr, s)
        _native.check(rc, "bs_zstd_decode")
    return d_src, d_dst, d_tasks, out_len, st, work


def _collect(issued):
    _, d_dst, _, out_len, st, _ = issued
    torch.cuda.synchronize()
    st.check("zstd")
    return [d.cpu().numpy().tobytes() for d in d_dst], out_len.cpu().tolist()


def _run(srcs, frames, static: bool):
    return _collect(_issue(_prepare(srcs, frames), static))


def test_static_scratch_entry_matches_work_buffer_entry():
    from bigsmall_amd import _native
    assert torch.cuda.is_available()
    for call, (seed, count, max_n) in enumerate([(1, 64, 300_000), (2, 9, 5_000)]):
        srcs, frames = _frames(seed, count, max_n)
        _say(f"[no-alloc] call {call + 1}: {count} frames, {sum(map(len, srcs))} bytes")
        got_s, len_s = _run(srcs, frames, static=True)
        got_w, len_w = _run(srcs, frames, static=False)
        assert len_s == len_w == [len(x) for x in srcs]
        for i, (a, b, src) in enumerate(zip(got_s, got_w, srcs)):
            assert a == b == src, (call, i)
    L = _native.lib()
    # two calls on two streams issued back to back, neither waited for before
    # the other is issued: the library orders them on the shared array, so
    # each decodes its own frames exactly
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    srcs1, frames1 = _frames(3, 48, 200_000)
    srcs2, frames2 = _frames(4, 40, 150_000)
    _say("[no-alloc] two calls on two streams")
    p1, p2 = _prepare(srcs1, frames1), _prepare(srcs2, frames2)
    i1 = _issue(p1, static=True, stream=a)
    i2 = _issue(p2, static=True, stream=b)
    for srcs, issued in ((srcs1, i1), (srcs2, i2)):
        got, lens = _collect(issued)
        assert lens == [len(x) for x in srcs]
        assert got == srcs
    too_many = _native.lib().bs_zstd_decode_static(1 << 12, 65, 1 << 12, 1 << 12, None)
    assert too_many == _native.BS_ERR_CAP
    assert L.bs_zstd_decode_static(0, 0, 0, 1 << 12, None) == _native.BS_OK
