"""GPU encoder for BSCK (bs_chunk_encode_gpu via bf16_chunked.encode_device).

Bar: every blob is byte-identical to the host encoder's blob for the same
words with the dense plane mode forced (encode_array(..., mode=MODE_DENSE,
lanes=128)), and decodes back to the source tensor bit-exactly. Covers chunk
edges (1 element, a partial step, exactly one chunk, one chunk plus one),
heavy tails, all-zero and single-exponent tensors, every exponent present,
several step counts, and batches mixing sizes (with an empty tensor).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _words(rng, kind: str, n: int) -> np.ndarray:
    if kind == "gauss":
        x = rng.standard_normal(n) * 0.02
    elif kind == "studentt":
        x = rng.standard_t(3, n) * 0.02
    elif kind == "kv":
        x = rng.standard_normal(n) * rng.uniform(0.5, 2.0)
    elif kind == "zeros":
        return np.zeros(n, np.uint16)
    elif kind == "one_exp":
        return (0x3F80 | rng.integers(0, 128, n) | (rng.integers(0, 2, n) << 15)).astype(np.uint16)
    elif kind == "uniform":
        return rng.integers(0, 65536, n).astype(np.uint16)
    else:
        raise ValueError(kind)
    return torch.from_numpy(x.astype(np.float32)).bfloat16().view(torch.int16).numpy().view(np.uint16)


def _check(words_list, steps):
    from bigsmall_amd.codecs import bf16_chunked as bc
    dev = torch.device("cuda", 0)
    ts = [torch.from_numpy(w.view(np.int16).copy()).view(torch.bfloat16).to(dev) for w in words_list]
    arena, spans = bc.encode_device(ts, steps=steps)
    host = arena.cpu().numpy()
    for w, (off, ln) in zip(words_list, spans):
        if w.size == 0:
            assert ln == 0
            continue
        want = bc.encode_array(w, steps=steps, mode=bc.MODE_DENSE, lanes=128)
        got = host[off:off + ln].tobytes()
        assert len(got) == len(want), (w.size, steps, len(got), len(want))
        assert got == want, (w.size, steps)
        out = torch.empty(w.size, dtype=torch.bfloat16, device=dev)
        st = bc.decode_into(arena[off:off + ln], ln, out, w.size)
        torch.cuda.synchronize()
        st.check("round trip")
        assert out.view(torch.int16).cpu().numpy().view(np.uint16).tobytes() == w.tobytes()


@pytest.mark.parametrize("steps", [16, 256, 448])
@pytest.mark.parametrize("n_rel", ["1", "127", "129", "per-1", "per", "per+1", "3per+17"])
def test_sizes_match_host_encoder(steps, n_rel):
    per = 128 * steps
    n = {"1": 1, "127": 127, "129": 129, "per-1": per - 1, "per": per, "per+1": per + 1,
         "3per+17": 3 * per + 17}[n_rel]
    rng = np.random.default_rng(n + steps)
    _say(f"[enc] gauss n={n} steps={steps}")
    _check([_words(rng, "gauss", n)], steps)


@pytest.mark.parametrize("kind", ["studentt", "kv", "zeros", "one_exp", "uniform"])
def test_distributions_match_host_encoder(kind):
    rng = np.random.default_rng(len(kind))
    _say(f"[enc] {kind} n=1000003")
    _check([_words(rng, kind, 1_000_003)], 256)


def test_batch_of_kv_blocks_and_mixed_sizes():
    rng = np.random.default_rng(11)
    ws = [_words(rng, "kv", 262_144) for _ in range(16)] + [np.zeros(0, np.uint16), _words(rng, "gauss", 5)]
    _say("[enc] batch of 18 tensors")
    _check(ws, 256)


def test_kv_cache_device_tensors_encode_on_gpu():
    """CompressedKVCache with K/V already in HBM: set_blocks and set encode on
    the GPU (dense-mode blobs equal to the host encoder's), get/get_blocks
    give the tensors back bit-exactly."""
    from bigsmall_amd.codecs import bf16_chunked as bc
    from bigsmall_amd.codecs import kv_cache as kvc
    from bigsmall_amd.kv_cache_manager import CompressedKVCache
    g = torch.Generator().manual_seed(21)
    s = torch.empty(8, 1, 1).uniform_(0.5, 2.0, generator=g)
    k = (torch.randn(8, 1024, 128, generator=g) * s).bfloat16()
    v = (torch.randn(8, 1024, 128, generator=g) * s).bfloat16()
    kd, vd = k.cuda(), v.cuda()
    c = CompressedKVCache(device="cuda")
    _say("[enc] kv set_blocks from device tensors")
    assert c.set_blocks(0, kd, vd, block_tokens=256) == 4
    L = c._blocks[0]
    host = L.arena.cpu().numpy()
    for b in range(4):
        off, ln, _, mode = L.k_blocks[b]
        words = k[:, b * 256:(b + 1) * 256].contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)
        assert host[off:off + ln].tobytes() == bc.encode_array(words, steps=kvc.KV_STEPS, mode=bc.MODE_DENSE, lanes=128)
    kb, vb = c.get_blocks(0, [2, 0, 3])
    for j, b in enumerate([2, 0, 3]):
        assert torch.equal(kb[j].cpu().view(torch.int16), k[:, b * 256:(b + 1) * 256].view(torch.int16))
        assert torch.equal(vb[j].cpu().view(torch.int16), v[:, b * 256:(b + 1) * 256].view(torch.int16))
    _say("[enc] kv set/get from device tensors")
    c.set(1, kd.unsqueeze(0), vd.unsqueeze(0))
    k2, v2 = c.get(1)
    assert torch.equal(k2.cpu().view(torch.int16), k.unsqueeze(0).view(torch.int16))
    assert torch.equal(v2.cpu().view(torch.int16), v.unsqueeze(0).view(torch.int16))
    assert 0.6 < c.compression_ratio() < 0.85


def test_encode_device_rows_matches_per_row_encoding():
    """encode_device_rows (the task table built per group, blobs packed by
    bs_copy_spans) gives every row the host encoder's dense-mode blob, packed
    back to back in row order; also on a side stream."""
    from bigsmall_amd.codecs import bf16_chunked as bc
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(31)
    shapes = [(12, 262_144), (0, 64), (5, 2), (3, 3 * 128 * 256 + 10)]
    words = [np.stack([_words(rng, "kv", n) for _ in range(r)]) if r else np.zeros((0, n), np.uint16)
             for r, n in shapes]
    groups = [torch.from_numpy(w.view(np.int16).copy()).view(torch.bfloat16).to(dev) for w in words]
    side = torch.cuda.Stream()
    for stream in (None, side):
        _say(f"[enc] rows, stream={'side' if stream else 'current'}")
        arena, offs, lens = bc.encode_device_rows(groups, steps=256, stream=stream)
        torch.cuda.synchronize()
        host = arena.cpu().numpy()
        rows = [w[i] for w in words for i in range(w.shape[0])]
        assert len(offs) == len(lens) == len(rows)
        pos = 0
        for w, off, ln in zip(rows, offs.tolist(), lens.tolist()):
            want = bc.encode_array(w, steps=256, mode=bc.MODE_DENSE, lanes=128)
            assert off == pos and ln == len(want)
            assert host[off:off + ln].tobytes() == want
            pos += ln


def test_copy_spans_packs_and_rejects_misaligned():
    """bs_copy_spans copies every 16-byte aligned span exactly, leaves bytes
    outside the spans alone, and flags (and skips) a misaligned span."""
    from bigsmall_amd import _native
    from bigsmall_amd.codecs import bf16_chunked as bc
    from bigsmall_amd.device import StatusWord, upload_bytes
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(5)
    src_h = rng.integers(0, 256, 4 << 20, dtype=np.uint8)
    src = torch.from_numpy(src_h).to(dev)
    dst = torch.full((4 << 20,), 0xAB, dtype=torch.uint8, device=dev)
    lens = [16, 32, 4096, 1 << 20, 48, 3 * 65536 + 16, 0]
    spans = np.zeros(len(lens) + 1, bc.SPAN_DTYPE)
    want = np.full(4 << 20, 0xAB, np.uint8)
    s_off, d_off = 0, 4 << 20           # sources ascending, destinations descending: no overlap
    for i, ln in enumerate(lens):
        d_off -= ln + 512
        d_off -= d_off % 16
        spans[i] = (src.data_ptr() + s_off, dst.data_ptr() + d_off, ln)
        want[d_off:d_off + ln] = src_h[s_off:s_off + ln]
        s_off += ln + 256
    assert s_off <= (4 << 20) and d_off >= 64
    spans[len(lens)] = (src.data_ptr() + 8, dst.data_ptr(), 32)          # misaligned src
    d_spans = upload_bytes(spans.view(np.uint8), dev)
    st = StatusWord(dev)
    _say("[enc] bs_copy_spans")
    _native.check(_native.lib().bs_copy_spans(d_spans.data_ptr(), len(spans), max(lens), st.ptr,
                                              torch.cuda.current_stream().cuda_stream), "bs_copy_spans")
    torch.cuda.synchronize()
    assert int(st.t.item()) == _native.BS_DEV_ERR_HEADER
    assert np.array_equal(dst.cpu().numpy(), want)


def test_kv_set_blocks_odd_block_size():
    """Blocks whose element count is odd (not 4-byte aligned rows) take the
    per-block-view encode path and still round-trip."""
    from bigsmall_amd.kv_cache_manager import CompressedKVCache
    g = torch.Generator().manual_seed(4)
    k = torch.randn(1, 514, 3, generator=g).bfloat16()
    v = torch.randn(1, 514, 3, generator=g).bfloat16()
    c = CompressedKVCache(device="cuda")
    _say("[enc] kv set_blocks with 771-element blocks")
    assert c.set_blocks(0, k.cuda(), v.cuda(), block_tokens=257) == 2
    kb, vb = c.get_blocks(0, [1, 0])
    for j, b in enumerate([1, 0]):
        assert torch.equal(kb[j].cpu().view(torch.int16), k[:, b * 257:(b + 1) * 257].view(torch.int16))
        assert torch.equal(vb[j].cpu().view(torch.int16), v[:, b * 257:(b + 1) * 257].view(torch.int16))


@pytest.mark.parametrize("where", ["before_plane", "in_plane", "after_plane"])
def test_capacity_too_small_reports_bounds_and_writes_nothing_past_it(where):
    """A task whose capacity is below its blob's length: BS_DEV_ERR_BOUNDS, a
    length of 0, and no byte at or past `cap` written. The capacity falls
    before the dense-plane region (the plan pass refuses), inside it (the
    chunk pass stores the full chunks' planes there and must skip them) or
    after it but short of the blob (the layout pass refuses)."""
    from bigsmall_amd import _native
    from bigsmall_amd.codecs import bf16_chunked as bc
    from bigsmall_amd.device import StatusWord, stream_ptr, upload_bytes
    dev = torch.device("cuda", 0)
    steps = 16
    per = 128 * steps
    nf = 5
    n = nf * per + 300                                   # five full chunks and a partial one
    nch = nf + 1
    w = _words(np.random.default_rng(7), "gauss", n)
    want = bc.encode_array(w, steps=steps, mode=bc.MODE_DENSE, lanes=128)
    nsym = int.from_bytes(want[22:24], "little")
    ctab = (32 + 4 * nsym + 15) & ~15
    preg = (ctab + 16 * nch + 255) & ~255
    cap = {"before_plane": preg - 16, "in_plane": preg + nf * per // 2, "after_plane": len(want) - 16}[where]
    assert preg + nf * per < len(want) - 16 and cap < len(want)
    _say(f"[encode cap] {where}: n={n} blob={len(want)} plane=[{preg}, {preg + nf * per}) cap={cap}")
    src = torch.from_numpy(w.view(np.int16).copy()).view(torch.bfloat16).to(dev)
    dst = torch.full((len(want) + 4096,), 0xAB, dtype=torch.uint8, device=dev)
    tasks = np.zeros(1, bc.ENCODE_TASK_DTYPE)
    tasks[0] = (src.data_ptr(), n, dst.data_ptr(), cap, 0, nch, 0, 0)
    d_tasks = upload_bytes(tasks.view(np.uint8), dev)
    L = _native.lib()
    wb = int(L.bs_chunk_encode_gpu_work_bytes(1, nch, steps))
    work = torch.empty(wb, dtype=torch.uint8, device=dev)
    out_len = torch.full((1,), -1, dtype=torch.int64, device=dev)
    st = StatusWord(dev)
    _native.check(L.bs_chunk_encode_gpu(d_tasks.data_ptr(), 1, nch, steps, work.data_ptr(), wb, out_len.data_ptr(),
                                        st.ptr, stream_ptr(None, dev)), "bs_chunk_encode_gpu")
    torch.cuda.synchronize()
    assert int(st.t.item()) & _native.BS_DEV_ERR_BOUNDS
    assert int(out_len.item()) == 0
    tail = dst[cap:].cpu().numpy()
    assert (tail == 0xAB).all(), f"{int((tail != 0xAB).sum())} bytes written at or past the capacity"


@pytest.mark.parametrize("steps,seg_len,nseg,pad", [(16, 512, 7, 24), (16, 3072, 3, 8), (32, 1536, 5, 16),
                                                   (256, 32768, 8, 0)])
def test_segmented_rows_match_contiguous_encoding(steps, seg_len, nseg, pad):
    """encode_device_rows on 3-D views [rows, segments, seg_len] (blocks of a
    [heads, tokens, dim] tensor read in place; bs_encode_task seg_len and
    seg_stride) writes the blobs the host encoder writes for each row copied
    to contiguous memory. The cases put full and partial chunks across
    segment boundaries, pad the segment stride, and start the segments 4 but
    not 16 bytes past an alignment boundary."""
    from bigsmall_amd.codecs import bf16_chunked as bc
    dev = torch.device("cuda", 0)
    rows, stride = 3, seg_len + pad
    g = torch.Generator().manual_seed(seg_len + nseg)
    flat = (torch.randn(nseg * rows * stride + 2, generator=g) * 0.05).bfloat16().to(dev)[2:]
    assert flat.data_ptr() % 16 == 4
    view = flat.view(nseg, rows, stride)[:, :, :seg_len].permute(1, 0, 2)     # [rows, nseg, seg_len]
    _say(f"[segmented] steps={steps} seg_len={seg_len} nseg={nseg} stride={stride} strides={view.stride()}")
    arena, offs, lens = bc.encode_device_rows([view], steps=steps)
    host = arena.cpu().numpy()
    for r in range(rows):
        words = view[r].contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
        want = bc.encode_array(words, steps=steps, mode=bc.MODE_DENSE, lanes=128)
        got = host[offs[r]:offs[r] + lens[r]].tobytes()
        assert got == want, (r, len(got), len(want))
    # a 2-D group in the same batch keeps its contiguous meaning
    plain = view[0].contiguous().reshape(1, -1)
    arena2, offs2, lens2 = bc.encode_device_rows([view, plain], steps=steps)
    h2 = arena2.cpu().numpy()
    assert h2[offs2[rows]:offs2[rows] + lens2[rows]].tobytes() == host[offs[0]:offs[0] + lens[0]].tobytes()


def test_segmented_rows_reject_bad_views():
    from bigsmall_amd.codecs import bf16_chunked as bc
    dev = torch.device("cuda", 0)
    x = torch.zeros(4, 3, 1024, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):                     # segments not a multiple of 512 words
        bc.encode_device_rows([x[:, :, :1000].permute(1, 0, 2)])
    with pytest.raises(ValueError):                     # segment starts not 8 words apart in multiples
        bc.encode_device_rows([torch.zeros(4 * 3 * 1028, dtype=torch.bfloat16, device=dev)
                               .view(4, 3, 1028)[:, :, :512].permute(1, 0, 2)])
