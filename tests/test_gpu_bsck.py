"""GPU parity of the BSCK (bf16_chunked_v1 / fp8_chunked_v1) HIP decoder.

Bar: bit-exact. Every case checks GPU output == source words (md5) and ==
the oracle's CPU decode of the same blob.
"""
from __future__ import annotations

import hashlib
import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _bf16(x: np.ndarray) -> np.ndarray:
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch_gpu():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    oracle.build()
    return torch


def _check_one(torch_gpu, words, steps=512, mode=-1, label="", lanes=128):
    from bigsmall_amd.codecs import bf16_chunked as bc
    _say(f"[bsck] {label} n={words.size} dtype={words.dtype} steps={steps} mode={mode} lanes={lanes}")
    blob = bc.encode_array(words, steps=steps, mode=mode, lanes=lanes)
    eb = words.dtype.itemsize
    gpu = bc.decode(blob, {}, words.size, elem_bytes=eb) if eb == 2 else bc.decode_fp8(blob, {}, words.size)
    assert hashlib.md5(gpu).hexdigest() == hashlib.md5(words.tobytes()).hexdigest(), label
    assert gpu == oracle.chunk_decode(blob, words.size, eb), label
    return blob


@pytest.mark.parametrize("lanes", [64, 128, 256])
@pytest.mark.parametrize("n", [1, 63, 64, 65, 127, 129, 511, 4097, 32768, 65536 * 3 + 1000, 1 << 20])
def test_gaussian_sizes(torch_gpu, n, lanes):
    rng = np.random.default_rng(n)
    _check_one(torch_gpu, _bf16(rng.standard_normal(n) * 0.02), label=f"gauss{n}", lanes=lanes)


@pytest.mark.parametrize("lanes", [64, 128, 256])
@pytest.mark.parametrize("mode", [-1, 1, 2])
@pytest.mark.parametrize("steps", [16, 64, 512, 1024])
def test_modes_and_steps(torch_gpu, mode, steps, lanes):
    rng = np.random.default_rng(steps + 7 * mode)
    w = _bf16(rng.standard_normal(200_003) * 0.02)
    w[rng.permutation(w.size)[: w.size // 2]] = 0          # 50% exact zeros (compact mode pays off)
    _check_one(torch_gpu, w, steps=steps, mode=mode, label=f"halfzero s{steps} m{mode}", lanes=lanes)


def test_edge_words_and_heavy_tails(torch_gpu):
    rng = np.random.default_rng(11)
    edge = np.array([0x7FC0, 0x7F80, 0xFF80, 0x0000, 0x8000, 0x0001, 0x0080, 0x3F80], np.uint16)
    w = np.concatenate([edge, _bf16(rng.standard_normal(100_000) * 0.02)])
    _check_one(torch_gpu, w, label="edge")
    t = _bf16(rng.standard_t(3, 300_000) * 0.02 / np.sqrt(3))
    _check_one(torch_gpu, t, label="student-t")
    allw = rng.integers(0, 65536, 300_000).astype(np.uint16)  # every exponent present
    _check_one(torch_gpu, allw, label="uniform words")        # ring refills take the slow path
    _check_one(torch_gpu, allw, label="uniform words k1", lanes=64)


def test_exact_value_modes(torch_gpu):
    rng = np.random.default_rng(12)
    _check_one(torch_gpu, np.zeros(100_000, np.uint16), label="zeros")
    _check_one(torch_gpu, _bf16(1.0 + rng.standard_normal(4096) * 0.01), label="norm")
    _check_one(torch_gpu, np.full(70_000, 0x3F80, np.uint16), mode=0, label="constant")
    fp8 = rng.integers(0, 256, 500_000).astype(np.uint8)
    _check_one(torch_gpu, fp8, label="fp8 uniform")
    _check_one(torch_gpu, fp8[:100_001], label="fp8 uniform k1", lanes=64)
    import torch
    x = torch.randn(300_000, generator=torch.Generator().manual_seed(5)).to(torch.float8_e4m3fn)
    _check_one(torch_gpu, x.view(torch.uint8).numpy(), label="fp8 e4m3 N(0,1)")


def test_batched_launch_matches_single(torch_gpu):
    import torch
    from bigsmall_amd.codecs import bf16_chunked as bc
    from bigsmall_amd.device import ChunkBatch, ChunkJob, StatusWord, upload_bytes
    rng = np.random.default_rng(13)
    sizes = [5, 64 * 512, 64 * 512 + 3, 1 << 18, 777_777]
    words = [_bf16(rng.standard_normal(s) * (0.01 + 0.01 * i)) for i, s in enumerate(sizes)]
    blobs = [bc.encode_array(w, lanes=(64, 128, 256)[i % 3]) for i, w in enumerate(words)]
    _say(f"[bsck] batch of {len(blobs)} blobs")
    dev = torch.device("cuda")
    d = [upload_bytes(b, dev) for b in blobs]
    outs = [torch.empty(w.size, dtype=torch.int16, device=dev) for w in words]
    jobs = [ChunkJob(db.data_ptr(), len(b), o.data_ptr(), w.size, bc.info(b).n_chunks, bc.info(b).plane_mode)
            for db, b, o, w in zip(d, blobs, outs, words)]
    st = StatusWord(dev)
    batch = ChunkBatch(jobs, dev)
    for rep in range(3):
        for o in outs:
            o.fill_(0)
        batch.launch(st)
        torch.cuda.synchronize()
        st.check()
        for o, w in zip(outs, words):
            assert np.array_equal(o.cpu().numpy().view(np.uint16), w), f"rep {rep}"


@pytest.mark.parametrize("n_tasks", [64, 65])
def test_batched_launch_at_the_task_lookup_boundary(torch_gpu, n_tasks):
    """A workgroup finds its task by rounds of a 64-way wavefront vote: up to
    64 tasks take the last round alone, 65 are the first count that needs a
    narrowing round before it (the next boundary, 4,096 / 4,097 tasks, runs
    in the CPU build of the kernel under AddressSanitizer). 64 and 65 blobs of
    one to three chunks each, the outputs in separate allocations so that
    their addresses differ in every bit range, each decoded bit-exact."""
    import torch
    from bigsmall_amd.codecs import bf16_chunked as bc
    from bigsmall_amd.device import ChunkBatch, ChunkJob, StatusWord, upload_bytes
    rng = np.random.default_rng(17 + n_tasks)
    words = [_bf16(rng.standard_normal(int(s)) * 0.02) for s in rng.integers(1, 3 * 8192, n_tasks)]
    blobs = [bc.encode_array(w, steps=64) for w in words]
    _say(f"[bsck] batch of {n_tasks} blobs")
    dev = torch.device("cuda")
    d = [upload_bytes(b, dev) for b in blobs]
    outs = [torch.empty(w.size, dtype=torch.int16, device=dev) for w in words]
    jobs = [ChunkJob(db.data_ptr(), len(b), o.data_ptr(), w.size, bc.info(b).n_chunks, bc.info(b).plane_mode)
            for db, b, o, w in zip(d, blobs, outs, words)]
    st = StatusWord(dev)
    batch = ChunkBatch(jobs, dev)
    for o in outs:
        o.fill_(0)
    batch.launch(st)
    torch.cuda.synchronize()
    st.check()
    for i, (o, w) in enumerate(zip(outs, words)):
        assert np.array_equal(o.cpu().numpy().view(np.uint16), w), f"task {i} of {n_tasks}"


def test_batched_launch_mixing_every_plane_mode(torch_gpu):
    """One launch holding compact (mode 2), dense (1) and exact (0) bf16 blobs
    and an fp8 blob, at every lane count, with partial last chunks: the
    compact launch decodes every mode with its own ring geometry."""
    import torch
    from bigsmall_amd.codecs import bf16_chunked as bc
    from bigsmall_amd.device import ChunkBatch, ChunkJob, StatusWord, upload_bytes
    rng = np.random.default_rng(15)
    cases = []
    for i, lanes in enumerate((64, 128, 256)):
        half = _bf16(rng.standard_normal(300_001 + 77 * i) * 0.02)
        half[rng.permutation(half.size)[: half.size // 2]] = 0
        cases.append((half, 2, lanes))
        cases.append((_bf16(rng.standard_normal(200_003) * 0.02), 1, lanes))
        cases.append((_bf16(1.0 + rng.standard_normal(70_001) * 0.01), 0, lanes))
        cases.append((rng.integers(0, 256, 150_007).astype(np.uint8), 0, lanes))
    blobs = [bc.encode_array(w, steps=64, mode=m, lanes=ln) for w, m, ln in cases]
    assert [bc.info(b).plane_mode for b in blobs] == [m for _, m, _ in cases]
    _say(f"[bsck] mixed-mode batch of {len(blobs)} blobs")
    dev = torch.device("cuda")
    d = [upload_bytes(b, dev) for b in blobs]
    outs = [torch.empty(w.nbytes, dtype=torch.uint8, device=dev) for w, _, _ in cases]
    jobs = [ChunkJob(db.data_ptr(), len(b), o.data_ptr(), w.size, bc.info(b).n_chunks, bc.info(b).plane_mode)
            for db, b, o, (w, _, _) in zip(d, blobs, outs, cases)]
    st = StatusWord(dev)
    batch = ChunkBatch(jobs, dev)
    for rep in range(2):
        for o in outs:
            o.fill_(0)
        batch.launch(st)
        torch.cuda.synchronize()
        st.check()
        for o, (w, m, ln) in zip(outs, cases):
            assert o.cpu().numpy().tobytes() == w.tobytes(), f"rep {rep} mode {m} lanes {ln} n {w.size}"


def test_concurrent_host_threads_on_their_own_streams(torch_gpu):
    """The C-ABI keeps no per-call global state: four host threads decode
    different blobs (BSCK dense, BSCK compact, a partial-chunk BSCK blob and the
    reference's bf16_parallel_v1) at once, each on its own stream, three rounds
    each, every result bit-exact."""
    import torch
    from concurrent.futures import ThreadPoolExecutor
    from bigsmall_amd.codecs import _refstreams
    from bigsmall_amd.codecs import bf16_chunked as bc
    rng = np.random.default_rng(16)
    dense = _bf16(rng.standard_normal(600_001) * 0.02)
    half = dense.copy()
    half[rng.permutation(half.size)[: half.size // 2]] = 0
    cases = [("bsck", bc.encode_array(dense, mode=1), dense),
             ("bsck", bc.encode_array(half, mode=2), half),
             ("bsck", bc.encode_array(dense[:77_777]), dense[:77_777]),
             ("par1", oracle.par1_encode(dense[:300_000]), dense[:300_000])]
    _say("[bsck] 4 host threads, one stream each")

    def work(i):
        kind, blob, w = cases[i]
        with torch.cuda.stream(torch.cuda.Stream()):
            for _ in range(3):
                got = (bc.decode(blob, {}, w.size) if kind == "bsck"
                       else _refstreams.decode_host("bf16_parallel_v1", blob, w.size))
                assert got == w.tobytes(), (i, kind)
        return i

    with ThreadPoolExecutor(4) as ex:
        assert sorted(ex.map(work, range(4))) == [0, 1, 2, 3]


@pytest.mark.parametrize("mode", [1, 2])
def test_single_byte_corruptions_decode_or_raise(torch_gpu, mode):
    """Every single-byte corruption of a blob (header, symbol table, chunk
    table, states, words, plane) either decodes or raises ValueError /
    DecodeError: the kernel's header, table and bounds checks keep every
    access inside the blob and the output, and most flips are reported."""
    import torch
    from bigsmall_amd.codecs import bf16_chunked as bc
    from bigsmall_amd.exceptions import DecodeError
    rng = np.random.default_rng(17 + mode)
    w = _bf16(rng.standard_normal(40_000) * 0.02)
    if mode == 2:
        w[rng.permutation(w.size)[: w.size // 2]] = 0
    blob = bc.encode_array(w, steps=64, mode=mode)
    ctab = (32 + 4 * int.from_bytes(blob[22:24], "little") + 15) & ~15
    head = list(range(0, ctab + 16 * bc.info(blob).n_chunks))       # header, symbols, chunk table
    positions = list(rng.choice(head, 80, replace=False)) + list(rng.integers(0, len(blob), 40))
    _say(f"[bsck] {len(positions) * 2} single-byte corruptions, mode {mode}")
    outcomes = {"ok": 0, "raised": 0}
    for pos in positions:
        for flip in (0xFF, 1 << int(rng.integers(0, 8))):
            bad = bytearray(blob)
            bad[pos] ^= flip
            try:
                bc.decode(bytes(bad), {}, w.size)
                outcomes["ok"] += 1
            except (ValueError, DecodeError):
                outcomes["raised"] += 1
    torch.cuda.synchronize()
    # the clean blob still decodes after all of them
    assert bc.decode(blob, {}, w.size) == w.tobytes()
    _say(f"[bsck] outcomes {outcomes}")
    assert outcomes["raised"] >= len(positions) // 2, outcomes


def test_corrupt_stream_is_reported(torch_gpu):
    import torch
    from bigsmall_amd.codecs import bf16_chunked as bc
    from bigsmall_amd.exceptions import DecodeError
    rng = np.random.default_rng(14)
    w = _bf16(rng.standard_normal(100_000) * 0.02)
    blob = bytearray(bc.encode_array(w))
    # flip one renorm word of chunk 0 (inside the blob, so every access stays in bounds)
    ctab = (32 + 4 * int.from_bytes(blob[22:24], "little") + 15) & ~15
    off = int.from_bytes(blob[ctab:ctab + 8], "little")
    blob[off + 256 + 10] ^= 0xFF
    _say("[bsck] corrupt word -> DecodeError")
    with pytest.raises(DecodeError):
        bc.decode(bytes(blob), {}, w.size)
    # wrong element count is refused on the host before any launch
    with pytest.raises(ValueError):
        bc.decode(bytes(blob), {}, w.size + 1)
    torch.cuda.synchronize()
