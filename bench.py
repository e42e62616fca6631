#!/usr/bin/env python3
"""Benchmark: decode one Llama-3-8B-shaped bf16 layer into HBM on one MI355X.

Workload (one "step" = one batched decode of the whole layer):
  q_proj/o_proj 4096x4096, k_proj/v_proj 1024x4096, gate/up 14336x4096,
  down 4096x14336, all N(0, 0.02) bf16 (torch CPU generator, seed 0), plus
  input_layernorm / post_attention_layernorm (1 + N(0, 0.01), length 4096).
  218,112,000 weights = 436,224,000 bytes of bf16. Every tensor is encoded with
  the engine's encoder (codec bf16_chunked_v1, auto mode). Six distinct layers
  (per-layer sign-flipped variants of the seeded draw) are uploaded to HBM once,
  each with its own preallocated bf16 outputs, and step i decodes all 9
  tensors of layer i mod 6 in ONE batched kernel launch: the timed working set
  (6 x 725 MB) is far beyond the 256 MB Infinity Cache, so no step is served
  from data an earlier step left there. Output is verified bit-exact (md5 per
  tensor, every layer) after the timed region. Before the W warm-up steps the
  layers are decoded untimed for --settle-ms (default 50 ms): from idle the
  GPU's clocks ramp over the first 15-20 ms of load, which a few warm-up steps
  do not cover.

Reported `value`: decoded GB/s counted as algorithmic bytes (compressed blob
bytes read + bf16 bytes written) per second. `roofline` uses HIP events
recorded on the launch stream around the timed launches; it also carries a
device-to-device copy measured in the same run (the practical ceiling for a
stream that reads and writes HBM). `cpu_baseline`: the oracle's C port of the
reference's fastest CPU decoder (bf16_se_single_kernel) on the same layer's
seven matrices, one host thread per tensor, with a single-thread figure beside it.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--settle-ms MS]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
WORKLOAD = "bsck_decode_llama3_8b_layer"
LAYER = [
    ("model.layers.0.self_attn.q_proj.weight", (4096, 4096)),
    ("model.layers.0.self_attn.k_proj.weight", (1024, 4096)),
    ("model.layers.0.self_attn.v_proj.weight", (1024, 4096)),
    ("model.layers.0.self_attn.o_proj.weight", (4096, 4096)),
    ("model.layers.0.mlp.gate_proj.weight", (14336, 4096)),
    ("model.layers.0.mlp.up_proj.weight", (14336, 4096)),
    ("model.layers.0.mlp.down_proj.weight", (4096, 14336)),
    ("model.layers.0.input_layernorm.weight", (4096,)),
    ("model.layers.0.post_attention_layernorm.weight", (4096,)),
]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_layer(seed: int = 0):
    import torch
    g = torch.Generator().manual_seed(seed)
    out = {}
    for name, shape in LAYER:
        if "norm" in name:
            t = 1.0 + torch.randn(shape, generator=g) * 0.01
        else:
            t = torch.randn(shape, generator=g) * 0.02
        out[name] = t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).reshape(-1)
    return out


def zero_layer(words: dict, fraction: float, seed: int = 1) -> dict:
    """The layer with a seeded Bernoulli(fraction) share of every matrix's
    elements set to +0.0 (a pruned model's layer); norms untouched."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, w in words.items():
        if "norm" not in name:
            w = w.copy()
            w[rng.random(w.size) < fraction] = 0
        out[name] = w
    return out


def host_cpu_info() -> dict:
    """The host CPU as /proc/cpuinfo names it (model name, family, model and
    stepping numbers, logical CPUs listed) and the CPUs this process may run on."""
    info = {}
    fields = {"model name": "cpu_model", "cpu family": "cpu_family", "model": "cpu_model_number",
              "stepping": "cpu_stepping", "cpu MHz": "cpu_mhz", "cache size": "cpu_cache"}
    listed = 0
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" not in line:
                    continue
                k, v = (x.strip() for x in line.split(":", 1))
                listed += k == "processor"
                if k in fields and fields[k] not in info:     # the first CPU's values
                    info[fields[k]] = v
    except OSError:
        pass
    info.setdefault("cpu_model", "unknown")
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    info["cpus_listed"] = listed
    info["host_cpus"] = usable
    return info


def _timed_cpu(fn, items) -> tuple[float, float]:
    """(algorithmic bytes, seconds) of fn over items, one after another."""
    t0 = time.perf_counter()
    done = sum(fn(it) for it in items)
    return done, time.perf_counter() - t0


def cpu_baseline(words: dict, budget_s: float = 6.0, bsck_blobs: dict | None = None):
    """The reference's CPU decode of the layer's seven matrices on the host
    cores (the oracle's C restatement, run without the GIL):
      value          bf16_parallel_v1 (bigsmall/codecs/bf16_parallel.py:262-352),
                     the reference's stream-parallel format: each matrix's 128
                     streams split over every host CPU, matrix after matrix;
      single_thread  the same on one thread, over the matrices that fit the
                     time budget;
      serial_chain   bf16_se_single_kernel (single_kernel.py:431-580), the
                     reference's fastest single-chain CPU decoder: one thread
                     per matrix (7) and one thread alone;
      same_format    the oracle's decoder of the blobs the GPU line decodes,
                     its chunks split over every host CPU, and on one thread."""
    from concurrent.futures import ThreadPoolExecutor
    import oracle
    oracle.build()
    host = host_cpu_info()
    cores = host["host_cpus"]
    mats = [(name, words[name]) for name, _ in LAYER if "norm" not in name]
    short = lambda names: ", ".join(nm.split(".")[-2] for nm in names)
    per_tensor = max(1, min(len(mats), cores, 16))
    with ThreadPoolExecutor(per_tensor) as ex:
        par1 = dict(zip([m[0] for m in mats], ex.map(lambda m: oracle.par1_encode(m[1]), mats)))
        sk = dict(zip([m[0] for m in mats], ex.map(lambda m: oracle.sk_encode(m[1]), mats)))

    def check(out, m, blob):
        assert out == m[1].tobytes(), f"oracle decode mismatch ({m[0]})"
        return m[1].nbytes + len(blob)

    # bf16_parallel_v1: every CPU on each matrix, then one thread on a budget
    par_all, t_par_all = _timed_cpu(lambda m: check(oracle.par1_decode_threads(par1[m[0]], m[1].size, cores), m,
                                                    par1[m[0]]), mats)
    done, t_one, names = 0, 0.0, []
    for m in mats:
        b, t = _timed_cpu(lambda mm: check(oracle.par1_decode(par1[mm[0]], mm[1].size), mm, par1[mm[0]]), [m])
        done, t_one = done + b, t_one + t
        names.append(m[0])
        if t_one > budget_s:
            break
    # bf16_se_single_kernel: one serial chain per matrix
    t0 = time.perf_counter()
    with ThreadPoolExecutor(per_tensor) as ex:
        sk_all = sum(ex.map(lambda m: check(oracle.sk_decode(sk[m[0]], m[1].size), m, sk[m[0]]), mats))
    t_sk_all = time.perf_counter() - t0
    sk_one, t_sk_one = _timed_cpu(lambda m: check(oracle.sk_decode(sk[m[0]], m[1].size), m, sk[m[0]]), mats[:2])
    out = {
        "value": par_all / t_par_all / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
        "sample": (f"oracle C port of the reference's bf16_parallel_v1 CPU decode (128 independent streams per "
                   f"tensor, split over {cores} host threads) of the layer's {len(mats)} matrices: "
                   f"{par_all / 1e6:.0f} MB algorithmic in {t_par_all:.2f} s"),
        "single_thread": {"value": done / t_one / 1e9, "unit": "GB/s", "cores": 1,
                          "sample": f"bf16_parallel_v1, {len(names)} tensors ({short(names)}): "
                                    f"{done / 1e6:.0f} MB algorithmic in {t_one:.2f} s"},
        "serial_chain": {"codec": "bf16_se_single_kernel", "value": sk_all / t_sk_all / 1e9, "unit": "GB/s",
                         "cores": per_tensor,
                         "sample": f"one host thread per tensor: {sk_all / 1e6:.0f} MB algorithmic in "
                                   f"{t_sk_all:.2f} s (one serial sign+exponent chain per tensor, so at most "
                                   f"one thread per tensor)",
                         "single_thread": {"value": sk_one / t_sk_one / 1e9, "cores": 1,
                                           "sample": f"{short([m[0] for m in mats[:2]])}: "
                                                     f"{sk_one / 1e6:.0f} MB algorithmic in {t_sk_one:.2f} s"}},
        "host": host,
    }
    if bsck_blobs is not None:
        bs_all, t_bs_all = _timed_cpu(lambda m: check(oracle.chunk_decode_threads(bsck_blobs[m[0]], m[1].size, cores),
                                                      m, bsck_blobs[m[0]]), mats)
        bs_one, t_bs_one = _timed_cpu(lambda m: check(oracle.chunk_decode(bsck_blobs[m[0]], m[1].size), m,
                                                      bsck_blobs[m[0]]), mats[:2])
        out["same_format"] = {
            "value": bs_all / t_bs_all / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": (f"the oracle's C decoder of the format the GPU line decodes on the layer's {len(mats)} "
                       f"matrices, chunks split over {cores} host threads: {bs_all / 1e6:.0f} MB algorithmic "
                       f"in {t_bs_all:.2f} s"),
            "single_thread": {"value": bs_one / t_bs_one / 1e9, "cores": 1,
                              "sample": f"{short([m[0] for m in mats[:2]])}: {bs_one / 1e6:.0f} MB algorithmic "
                                        f"in {t_bs_one:.2f} s"}}
    return out


def measure_copy(dev, mib: int = 2048, reps: int = 10) -> float:
    """Device-to-device copy rate in the same run, (read + write) bytes per
    second: the practical ceiling for a stream that reads and writes HBM. 2 GiB
    each way, far beyond the 256 MB Infinity Cache, so no pass is served from it."""
    import torch
    n = mib << 20
    a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    b.copy_(a)
    s = torch.cuda.current_stream(dev)
    ms = _timed(lambda: b.copy_(a), reps, s)
    del a, b
    return 2 * n / (ms * 1e-3) / 1e9


def hbm_probe(dev, mib: int = 2048, reps: int = 10) -> dict:
    """HBM rates by direction over 2 GiB buffers (far beyond the Infinity
    Cache): a read-only stream (torch's int64 sum), a write-only stream
    (torch's fill_) and read + write copies (torch's copy_ and this library's
    bs_copy_spans), in GB/s of bytes moved. A stream that both reads and
    writes, as a decode does, runs below either direction alone."""
    import torch
    n = mib << 20
    a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    s = torch.cuda.current_stream(dev)
    a64 = a.view(torch.int64)
    out = {}
    for name, fn, moved in (("read_only_sum", lambda: a64.sum(), n), ("write_only_fill", lambda: b.fill_(3), n),
                            ("copy_torch", lambda: b.copy_(a), 2 * n)):
        fn()
        out[name] = round(moved / (_timed(fn, reps, s) * 1e-3) / 1e9, 1)
    del a, b, a64
    out["copy_bs_copy_spans"] = round(measure_copy_kernel(dev, mib, reps), 1)
    log(f"[hbm] read-only {out['read_only_sum']:.0f} GB/s, write-only {out['write_only_fill']:.0f} GB/s, "
        f"copy {out['copy_torch']:.0f} (torch) / {out['copy_bs_copy_spans']:.0f} (bs_copy_spans) GB/s")
    return {"workload": "hbm_probe", "bytes_each": n, "unit": "GB/s", **out}


def measure_copy_kernel(dev, mib: int = 2048, reps: int = 10) -> float:
    """The same copy by this library's own copy kernel (bs_copy_spans, one
    span: four 16-byte vectors per lane, streaming loads and stores), (read +
    write) bytes per second."""
    import torch
    from bigsmall_amd import _native
    from bigsmall_amd.codecs.bf16_chunked import SPAN_DTYPE
    from bigsmall_amd.device import StatusWord, upload_bytes
    n = mib << 20
    a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    span = np.zeros(1, SPAN_DTYPE)
    span[0] = (a.data_ptr(), b.data_ptr(), n)
    d_span = upload_bytes(span.view(np.uint8), dev)
    st = StatusWord(dev)
    s = torch.cuda.current_stream(dev)
    L = _native.lib()
    fn = lambda: _native.check(L.bs_copy_spans(d_span.data_ptr(), 1, n, st.ptr, s.cuda_stream), "bs_copy_spans")
    fn()
    ms = _timed(fn, reps, s)
    st.check("copy kernel")
    assert torch.equal(a[:: 1 << 20], b[:: 1 << 20])
    del a, b
    return 2 * n / (ms * 1e-3) / 1e9


def copy_probe(mib: int) -> None:
    """A plain copy of known size: each launch reads and writes mib MiB. Its
    FETCH_SIZE / WRITE_SIZE readings calibrate the counters for `traffic`."""
    import torch
    n = mib << 20
    a = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": n, "launches": 3}), flush=True)


def measured_traffic(workload: str):
    """HBM bytes per launch of the decode kernel from the committed rocprofv3
    counter summary (FETCH_SIZE + WRITE_SIZE, calibrated against a plain copy),
    or None when no summary for this workload is committed."""
    path = os.path.join(ROOT, "profiles", f"{workload}.traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    return int(t["fetch_bytes_per_launch"] + t["write_bytes_per_launch"])


def _variants(base: np.ndarray, i: int) -> np.ndarray:
    """Per-layer variant of a seeded draw: flip each sign bit with a seeded
    coin. Same distribution (N(0, s) is symmetric), different data per layer.
    Exact zeros stay +0.0, as a pruned layer holds them."""
    flips = np.random.default_rng(1000 + i).integers(0, 2, base.size, dtype=np.uint16) << 15
    return base ^ (flips * (base != 0)).astype(np.uint16)


def settle(fn, ms: float) -> int:
    """Run `fn` (one step of the workload) untimed for `ms` milliseconds of
    wall time before the warm-up steps; returns the steps run. From idle the
    GPU raises its clocks over the first 15-20 ms of sustained load: the
    layer decode took 176 us per launch over its first 25 launches, 159 over
    the next 25, and settled at 144 us after about 100 (per-launch HIP events,
    one process), so a throughput figure taken over a few warm-up and 20
    timed launches would time the ramp rather than the decode."""
    import torch
    n, t0 = 0, time.perf_counter()
    while ms > 0 and (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(8):
            fn()
        n += 8
        torch.cuda.synchronize()
    return n


def _timed(fn, steps: int, stream):
    import torch
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(stream)
    for _ in range(steps):
        fn()
    ev1.record(stream)
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / steps


def _verify_device(outs: dict, tensors: list, dev, what: str) -> None:
    """Every decoded tensor equals its source words, compared on the device
    (each source uploaded in turn); raises on the first mismatch."""
    import torch
    for name, w in tensors:
        src = torch.from_numpy(w.view(np.int16)).to(dev)
        if not torch.equal(outs[name].view(torch.int16), src):
            raise AssertionError(f"{what}: {name} differs from its source")
        del src
    log(f"[{what}] all {len(tensors)} tensors bit-exact")


def run_model(args) -> dict:
    """Full Llama-3-8B-shaped model (32 layers + embed_tokens + lm_head, 128256x4096):
    decode every tensor into HBM. Reports decode from HBM-resident compressed
    layers (one batched launch per layer) and, separately, the end-to-end time
    with the compressed bytes copied host->device from pinned memory by the
    engine's layer pipeline (copy of layer i+1 overlapping decode of layer i)."""
    import torch
    from bigsmall_amd.codecs import bf16_chunked as bc
    from bigsmall_amd.device import ChunkBatch, ChunkJob, StatusWord
    t0 = time.time()
    base_layer = make_layer(0)
    g = torch.Generator().manual_seed(1)
    emb = (torch.randn(128256 * 4096, generator=g) * 0.02).bfloat16().view(torch.int16).numpy().view(np.uint16)
    tensors = [("model.embed_tokens.weight", emb)]
    for i in range(32):
        for name, w in base_layer.items():
            tensors.append((name.replace("layers.0.", f"layers.{i}."), w if "norm" in name else _variants(w, i)))
    tensors.append(("lm_head.weight", _variants(emb, 99)))
    log(f"[model] generated {len(tensors)} tensors in {time.time() - t0:.1f}s")
    t0 = time.time()
    data = bytearray()
    entries = []
    for name, w in tensors:
        blob = bc.encode_array(w)
        data += b"\x00" * ((-len(data)) % 256)
        info = bc.info(blob)
        entries.append({"name": name, "shape": [int(w.size)], "dtype": "bfloat16", "codec": bc.CODEC_BF16,
                        "offset": len(data), "compressed_bytes": len(blob), "extra": None,
                        "n_chunks": info.n_chunks, "plane_mode": info.plane_mode})
        data += blob
    host = np.frombuffer(data, np.uint8)
    n_total = sum(w.size for _, w in tensors)
    comp_total = sum(e["compressed_bytes"] for e in entries)
    log(f"[model] encoded {n_total / 1e9:.2f} G weights -> {comp_total / 1e9:.2f} GB in {time.time() - t0:.1f}s")
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    # (1) decode-only: compressed model resident in HBM, one batched launch per layer group
    d_all = torch.from_numpy(host).to(dev)
    outs = {e["name"]: torch.empty(int(e["shape"][0]), dtype=torch.bfloat16, device=dev) for e in entries}
    from bigsmall_amd.decoder import layer_groups
    groups = layer_groups(entries)
    batches = [ChunkBatch([ChunkJob(d_all.data_ptr() + e["offset"], e["compressed_bytes"],
                                    outs[e["name"]].data_ptr(), int(e["shape"][0]), e["n_chunks"], e["plane_mode"])
                           for e in grp], dev) for grp in groups]
    st = StatusWord(dev)
    # consecutive groups alternate between two streams, as the engine's
    # GroupDecoder issues them (a group's prologue under the previous one's tail)
    alt = torch.cuda.Stream(dev)

    def run_all():
        fork = torch.cuda.Event()
        fork.record(stream)
        alt.wait_event(fork)
        for i, b in enumerate(batches):
            b.launch(st, (stream, alt)[i % 2])
        join = torch.cuda.Event()
        join.record(alt)
        stream.wait_event(join)
    settle(run_all, args.settle_ms)
    run_all()
    torch.cuda.synchronize()
    st.check("model warmup")
    ms = _timed(run_all, max(1, args.steps // 10), stream)
    st.check("model timed")
    algo = comp_total + 2 * n_total
    _verify_device(outs, tensors, dev, "model decode")
    del outs, d_all
    torch.cuda.empty_cache()
    # (2) end-to-end from pinned host memory: per layer group, a host->device
    # copy on a copy stream and the group's batched decode waiting on it only,
    # so the copy of group g+1 overlaps the decode of group g
    outs = {e["name"]: torch.empty(int(e["shape"][0]), dtype=torch.bfloat16, device=dev) for e in entries}
    pinned = torch.from_numpy(host).pin_memory()
    copy_stream = torch.cuda.Stream(dev)
    plan = []
    for grp in groups:
        lo = min(e["offset"] for e in grp)
        hi = max(e["offset"] + e["compressed_bytes"] for e in grp)
        d = torch.empty(hi - lo, dtype=torch.uint8, device=dev)
        b = ChunkBatch([ChunkJob(d.data_ptr() + e["offset"] - lo, e["compressed_bytes"], outs[e["name"]].data_ptr(),
                                 int(e["shape"][0]), e["n_chunks"], e["plane_mode"]) for e in grp], dev)
        plan.append((lo, hi, d, b, torch.cuda.Event()))

    def e2e():
        for i, (lo, hi, d, b, ev) in enumerate(plan):
            with torch.cuda.stream(copy_stream):
                d.copy_(pinned[lo:hi], non_blocking=True)
                ev.record(copy_stream)
            s = (stream, alt)[i % 2]
            s.wait_event(ev)
            b.launch(st, s)
        torch.cuda.synchronize()
    e2e()
    t0 = time.perf_counter()
    e2e()
    e2e_s = time.perf_counter() - t0
    st.check("model e2e")
    _verify_device(outs, tensors, dev, "model end to end")
    return {"metric": "decoded bf16 GB/s, full Llama-3-8B-shaped model (decode from HBM)",
            "value": round(algo / (ms * 1e-3) / 1e9, 2), "unit": "GB/s", "n_gpus": 1,
            "ms_per_step": round(ms, 4), "higher_is_better": True, "dtype": "u32", "settle_ms": args.settle_ms,
            "data": "synthetic: seeded N(0,0.02) layer + embedding draws, per-layer sign-flipped variants",
            "config": {"workload": "bsck_decode_llama3_8b_model", "tensors": len(tensors), "elements": int(n_total),
                       "compressed_bytes": int(comp_total), "decoded_bytes": int(2 * n_total),
                       "ratio_pct": round(100 * comp_total / (2 * n_total), 3), "launches_per_step": len(batches)},
            "roofline": {"bound": "hbm", "achieved": round(algo / (ms * 1e-3) / 1e9, 2), "peak": HBM_PEAK_GBPS,
                         "unit": "GB/s", "frac": round(algo / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)},
            "end_to_end_from_pinned_host": {"seconds": round(e2e_s, 4),
                                            "compressed_GBps_over_pcie": round(comp_total / e2e_s / 1e9, 2),
                                            "decoded_GBps": round(2 * n_total / e2e_s / 1e9, 2)}}


def run_kv(args) -> dict:
    """KV-cache blocks: K and V [32 layers, 8 heads, 32768 tokens, 128] bf16,
    N(0, 1) scaled per head by U[0.5, 2], compressed in 256-token blocks; 64
    random blocks per layer (K and V) decoded in one launch."""
    import torch
    from bigsmall_amd.device import StatusWord
    from bigsmall_amd.kv_cache_manager import CompressedKVCache
    t0 = time.time()
    g = torch.Generator().manual_seed(2)
    s = torch.empty(8, 1, 1).uniform_(0.5, 2.0, generator=g)
    k0 = (torch.randn(8, 32768, 128, generator=g) * s).bfloat16()
    v0 = (torch.randn(8, 32768, 128, generator=g) * s).bfloat16()
    kw = k0.view(torch.int16).numpy().view(np.uint16).reshape(-1)
    vw = v0.view(torch.int16).numpy().view(np.uint16).reshape(-1)
    cache = CompressedKVCache(device="cuda")
    src = {}
    dev_kv = []
    for layer in range(32):
        k = torch.from_numpy(_variants(kw, 2 * layer).view(np.int16)).view(torch.bfloat16).reshape(8, 32768, 128)
        v = torch.from_numpy(_variants(vw, 2 * layer + 1).view(np.int16)).view(torch.bfloat16).reshape(8, 32768, 128)
        dev_kv.append((k.cuda(), v.cuda()))
        if layer < 2:
            src[layer] = (k, v)
    log(f"[kv] generated 32 layers in {time.time() - t0:.1f}s")
    # K/V already in HBM: set_blocks encodes on the GPU (timed, synchronous per layer)
    cache.set_blocks(0, *dev_kv[0], block_tokens=256)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for layer in range(32):
        cache.set_blocks(layer, *dev_kv[layer], block_tokens=256)
    torch.cuda.synchronize()
    enc_s = time.perf_counter() - t0
    raw_kv = 32 * 2 * k0.numel() * 2
    log(f"[kv] GPU-encoded 32 layers in {enc_s * 1e3:.1f} ms ({raw_kv / enc_s / 1e9:.1f} GB/s raw), "
        f"ratio {cache.compression_ratio():.4f}")
    # the same 32 layers set again: each replaces its layer, so the allocator
    # reuses the freed blocks instead of mapping new memory
    t0 = time.perf_counter()
    for layer in range(32):
        cache.set_blocks(layer, *dev_kv[layer], block_tokens=256)
    torch.cuda.synchronize()
    reenc_s = time.perf_counter() - t0
    log(f"[kv] re-encoded 32 layers in place in {reenc_s * 1e3:.1f} ms ({raw_kv / reenc_s / 1e9:.1f} GB/s raw)")
    # the path without the GPU encoder, for comparison: device K/V copied to the
    # host and encoded by the multithreaded C++ encoder (two layers)
    from bigsmall_amd.codecs.bf16_chunked import _threads as bc_threads
    host_cache = CompressedKVCache(device="cuda")
    t0 = time.perf_counter()
    for layer in range(2):
        host_cache.set_blocks(layer, dev_kv[layer][0].cpu(), dev_kv[layer][1].cpu(), block_tokens=256)
    torch.cuda.synchronize()
    host_s = (time.perf_counter() - t0) / 2
    raw_layer = 2 * k0.numel() * 2
    log(f"[kv] host path (D2H + C++ encode + upload): {host_s * 1e3:.1f} ms per layer "
        f"({raw_layer / host_s / 1e9:.2f} GB/s raw)")
    del host_cache
    rng = np.random.default_rng(3)
    req = [(layer, rng.choice(128, 64, replace=False)) for layer in range(32)]
    batch, outs = cache.prepare_blocks_multi(req)
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    st = StatusWord(dev)
    settle(lambda: batch.launch(st, stream), args.settle_ms)
    batch.launch(st, stream)
    torch.cuda.synchronize()
    st.check("kv warmup")
    ms = _timed(lambda: batch.launch(st, stream), args.steps, stream)
    st.check("kv timed")
    # every decoded block against its source, on the device: [8, 128 blocks, 256, 128] -> the requested blocks
    for layer in range(32):
        ids = torch.as_tensor(req[layer][1], dtype=torch.long, device=dev)
        for which in range(2):
            want = dev_kv[layer][which].view(8, 128, 256, 128).index_select(1, ids).movedim(1, 0)
            if not torch.equal(outs[layer][which], want):
                raise AssertionError(f"kv: layer {layer} {'KV'[which]} blocks differ from the source")
    log(f"[kv] all {len(batch.jobs)} decoded blocks bit-exact")
    for layer in range(2):     # and two layers against the host copies the device K/V came from
        k, v = src[layer]
        for j, b in enumerate(req[layer][1][:4]):
            assert torch.equal(outs[layer][0][j].cpu(), k[:, b * 256:(b + 1) * 256]), (layer, j)
            assert torch.equal(outs[layer][1][j].cpu(), v[:, b * 256:(b + 1) * 256]), (layer, j)
    del dev_kv
    comp = sum(job.blob_bytes for job in batch.jobs)
    out_bytes = sum(job.n for job in batch.jobs) * 2
    gbps = (comp + out_bytes) / (ms * 1e-3) / 1e9
    return {"metric": "decoded bf16 GB/s, KV-cache block decompression (64 random 256-token blocks x 32 layers x K,V)",
            "value": round(gbps, 2), "unit": "GB/s", "n_gpus": 1, "ms_per_step": round(ms, 4),
            "higher_is_better": True, "dtype": "u32", "settle_ms": args.settle_ms,
            "data": "synthetic: seeded N(0,1) x U[0.5,2] per head, per-layer sign-flipped variants",
            "config": {"workload": "bsck_kv_blocks_32x64", "blobs": len(batch.jobs), "compressed_bytes": int(comp),
                       "decoded_bytes": int(out_bytes), "ratio_pct": round(100 * cache.compression_ratio(), 3),
                       "launches_per_step": 1},
            "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4)},
            "gpu_encode": {"seconds_32_layers": round(enc_s, 4), "raw_GBps": round(raw_kv / enc_s / 1e9, 2),
                           "seconds_32_layers_in_place": round(reenc_s, 4),
                           "raw_GBps_in_place": round(raw_kv / reenc_s / 1e9, 2),
                           "note": "CompressedKVCache.set_blocks on device K/V, incl. block-major copies and "
                                   "blob packing; the first figure fills an empty cache (new device memory "
                                   "per layer), the second sets the same layers again"},
            "host_path_encode": {"seconds_per_layer": round(host_s, 4), "raw_GBps": round(raw_layer / host_s / 1e9, 3),
                                 "threads": bc_threads(),
                                 "note": "set_blocks on host copies of the device K/V (D2H + C++ encoder + upload)"}}


def cpu_baseline_refcodecs(words: np.ndarray) -> dict:
    """The reference's formats on the C0 tensor: blobs written by the oracle's
    encoders (byte-identical to the reference's, pinned by the golden
    fixtures) and the oracle's C decoders timed on one host thread."""
    import oracle
    oracle.build()
    out = {}
    for codec, enc, dec in (("bf16_parallel_v1", oracle.par1_encode, oracle.par1_decode),
                            ("bf16_se_tans", oracle.tans_encode, oracle.tans_decode),
                            ("bf16_se_single_kernel", oracle.sk_encode, oracle.sk_decode)):
        blob = enc(words)
        t0 = time.perf_counter()
        got = dec(blob, words.size)
        dt = time.perf_counter() - t0
        assert got == words.tobytes(), codec
        out[codec] = (blob, (len(blob) + words.nbytes) / dt / 1e9)
    return out


def run_refcodecs(args) -> dict:
    """C0 (4096x4096 N(0, 0.02) bf16, seed 0) in the reference's own formats,
    decoded on the GPU (bs_refcodec_decode / bs_refcodec_decode_serial) from an
    HBM-resident blob, beside the oracle's single-thread C decoder."""
    import torch
    from bigsmall_amd.codecs import _refstreams
    from bigsmall_amd.device import StatusWord, upload_bytes
    g = torch.Generator().manual_seed(0)
    words = (torch.randn(4096 * 4096, generator=g) * 0.02).bfloat16().view(torch.int16).numpy().view(np.uint16)
    base = cpu_baseline_refcodecs(words)
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    res = {}
    for codec, (blob, cpu_gbps) in base.items():
        d_blob = upload_bytes(blob, dev)
        out = torch.empty(words.size, dtype=torch.int16, device=dev)
        st = StatusWord(dev)
        launch = _refstreams.RefLaunch(_refstreams.PARSERS[codec](blob, words.size), d_blob.data_ptr(), dev,
                                       out.data_ptr())
        fn = lambda: launch.launch(out.data_ptr(), st.ptr, stream.cuda_stream)
        fn()
        torch.cuda.synchronize()
        st.check(codec)
        reps = 10 if codec == "bf16_parallel_v1" else 2
        ms = _timed(fn, reps, stream)
        st.check(codec)
        assert out.cpu().numpy().view(np.uint16).tobytes() == words.tobytes(), codec
        gbps = (len(blob) + words.nbytes) / (ms * 1e-3) / 1e9
        res[codec] = {"ms": round(ms, 3), "GBps": round(gbps, 3), "ratio_pct": round(100 * len(blob) / words.nbytes, 3),
                      "cpu_baseline_GBps_1_thread": round(cpu_gbps, 4), "gpu_over_cpu": round(gbps / cpu_gbps, 2)}
        log(f"[ref] {codec}: {ms:.2f} ms on GPU ({gbps:.3f} GB/s), oracle CPU {cpu_gbps:.3f} GB/s")
    return {"metric": "decoded GB/s of the reference's bf16 formats on 1 MI355X (C0 tensor)",
            "value": res["bf16_parallel_v1"]["GBps"], "unit": "GB/s", "n_gpus": 1,
            "ms_per_step": res["bf16_parallel_v1"]["ms"], "higher_is_better": True, "dtype": "u32",
            "data": "synthetic: torch seed 0, randn(4096*4096)*0.02 -> bf16; blobs byte-identical to the reference's",
            "host": host_cpu_info(), "config": {"workload": "refcodecs_c0_4096sq", "elements": int(words.size)},
            "codecs": res,
            "roofline": {"bound": "latency (serial rANS chains: 128 streams for bf16_parallel_v1, one for the others)",
                         "achieved": res["bf16_parallel_v1"]["GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(res["bf16_parallel_v1"]["GBps"] / HBM_PEAK_GBPS, 5)}}


def run_reflayer(args) -> dict:
    """The Llama-3-8B-shaped layer's seven matrices (seed 0, as the headline)
    written in the reference's own formats (bf16_parallel_v1 and bf16_se_tans,
    by the oracle's encoders, byte-identical to the reference's) and decoded
    on the GPU from HBM: all seven tensors in one bs_refcodec_decode_serial_batch
    launch (their chains side by side), beside one launch per tensor in turn,
    and beside the oracle's C decoders on the host (one thread per tensor)."""
    from concurrent.futures import ThreadPoolExecutor
    import torch
    import oracle
    from bigsmall_amd.codecs import _refstreams
    from bigsmall_amd.device import StatusWord, upload_bytes
    oracle.build()
    words = make_layer(0)
    mats = [(name, words[name]) for name, _ in LAYER if "norm" not in name]
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    res = {}
    codecs = (("bf16_parallel_v1", oracle.par1_encode, oracle.par1_decode),
              ("bf16_se_tans", oracle.tans_encode, oracle.tans_decode))
    if args.ref_codecs:
        codecs = tuple(c for c in codecs if c[0] in args.ref_codecs.split(","))
    for codec, enc, dec in codecs:
        t0 = time.time()
        with ThreadPoolExecutor(len(mats)) as ex:
            blobs = list(ex.map(lambda m: enc(m[1]), mats))
        log(f"[reflayer] {codec}: encoded in {time.time() - t0:.1f}s")
        algo = sum(len(b) + w.nbytes for b, (_, w) in zip(blobs, mats))
        d_blobs = [upload_bytes(b, dev) for b in blobs]
        outs = [torch.empty(w.size, dtype=torch.int16, device=dev) for _, w in mats]
        plans = [_refstreams.PARSERS[codec](b, w.size) for b, (_, w) in zip(blobs, mats)]
        st = StatusWord(dev)
        batch = _refstreams.RefBatch([(p, d.data_ptr(), o.data_ptr()) for p, d, o in zip(plans, d_blobs, outs)], dev)
        fn = lambda: batch.launch(st.ptr, stream.cuda_stream)
        fn()
        torch.cuda.synchronize()
        st.check(codec)
        reps = 3 if codec == "bf16_parallel_v1" else 1
        ms_batch = _timed(fn, reps, stream)
        st.check(codec)
        for o, (name, w) in zip(outs, mats):
            assert o.cpu().numpy().view(np.uint16).tobytes() == w.tobytes(), (codec, name)
        singles = [_refstreams.RefLaunch(p, d.data_ptr(), dev, o.data_ptr()) for p, d, o in zip(plans, d_blobs, outs)]
        seq = lambda: [l.launch(o.data_ptr(), st.ptr, stream.cuda_stream) for l, o in zip(singles, outs)]
        ms_seq = _timed(seq, 1, stream)
        st.check(codec)
        for o, (name, w) in zip(outs, mats):
            assert o.cpu().numpy().view(np.uint16).tobytes() == w.tobytes(), (codec, name)
        del singles
        t0 = time.perf_counter()
        with ThreadPoolExecutor(len(mats)) as ex:
            oks = list(ex.map(lambda bm: dec(bm[0], bm[1][1].size) == bm[1][1].tobytes(), zip(blobs, mats)))
        cpu_s = time.perf_counter() - t0
        assert all(oks), codec
        res[codec] = {"ms_one_batched_launch": round(ms_batch, 2), "ms_per_tensor_launches": round(ms_seq, 2),
                      "GBps": round(algo / (ms_batch * 1e-3) / 1e9, 3),
                      "ratio_pct": round(100 * sum(len(b) for b in blobs) / (2 * sum(w.size for _, w in mats)), 3),
                      "cpu_baseline": {"seconds": round(cpu_s, 3), "GBps": round(algo / cpu_s / 1e9, 3),
                                       "cores": len(mats), "kind": "port",
                                       "sample": "the oracle's C decoder of this format on the same seven blobs, "
                                                 "one host thread per tensor"}}
        log(f"[reflayer] {codec}: batch {ms_batch:.1f} ms, per-tensor launches {ms_seq:.1f} ms, "
            f"oracle CPU ({len(mats)} threads) {cpu_s * 1e3:.0f} ms")
        del d_blobs, outs, batch
    head = res[next(iter(res))]
    return {"metric": "ms per Llama-3-8B-shaped layer written in the reference's own formats, decoded on 1 MI355X",
            "value": head["ms_one_batched_launch"], "unit": "ms/layer", "n_gpus": 1,
            "ms_per_step": head["ms_one_batched_launch"], "higher_is_better": False, "dtype": "u32",
            "data": "synthetic: the headline layer's seven matrices (seed 0); blobs byte-identical to the reference's",
            "host": host_cpu_info(), "config": {"workload": "refcodecs_llama3_8b_layer", "tensors": len(mats)},
            "codecs": res,
            "roofline": {"bound": "latency (serial rANS chains: 128 per tensor for bf16_parallel_v1, one for "
                                  "bf16_se_tans)", "achieved": head["GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(head["GBps"] / HBM_PEAK_GBPS, 5)}}


def _c3_tensors():
    """8192x8192 stress tensors: (a) Student-t df=3 at std 0.02, (b) N(0, 0.02)
    with exactly half the positions (randperm) +0.0, (c) fp8 e4m3 of N(0, 1)
    and its bf16 residual."""
    import torch
    n = 8192 * 8192
    g = torch.Generator().manual_seed(3)
    # Student-t with 3 degrees of freedom from the seeded generator: Z / sqrt(chi2_3 / 3),
    # chi2_3 a sum of three squared standard normals (std of t_3 is sqrt(3))
    z = torch.randn(n, generator=g)
    chi2 = sum(torch.randn(n, generator=g) ** 2 for _ in range(3))
    st = (z / torch.sqrt(chi2 / 3.0) * (0.02 / np.sqrt(3.0))).bfloat16()
    hz = (torch.randn(n, generator=g) * 0.02).bfloat16()
    hz[torch.randperm(n, generator=g)[: n // 2]] = 0
    x = torch.randn(n, generator=torch.Generator().manual_seed(4))
    f8 = x.to(torch.float8_e4m3fn)
    resid = (x - f8.float()).bfloat16()
    w = lambda t: t.view(torch.int16).numpy().view(np.uint16)
    return [("studentt", w(st)), ("halfzero", w(hz)), ("fp8_e4m3", f8.view(torch.uint8).numpy()),
            ("fp8_residual", w(resid))]


def cpu_baseline_c3(tensors) -> dict:
    """bf16_se_tans (the reference's forced-tANS codec) blobs from the oracle's
    encoder, and its C decoder timed on one host thread."""
    import oracle
    oracle.build()
    out = {}
    for name, w in tensors:
        if w.dtype != np.uint16:
            continue
        blob = oracle.tans_encode(w)
        t0 = time.perf_counter()
        assert oracle.tans_decode(blob, w.size) == w.tobytes(), name
        out[name] = (blob, (len(blob) + w.nbytes) / (time.perf_counter() - t0) / 1e9)
    return out


def run_c3(args) -> dict:
    """The 8192x8192 stress tensors decoded on the GPU, one launch per tensor:
    forced rANS = this engine's bf16_chunked_v1 / fp8_chunked_v1 and forced
    tANS = its bf16_chunked_tans_v1 / fp8_chunked_tans_v1 (fp8 as exponent
    pairs, the automatic choice); beside them the reference's forced-tANS
    format bf16_se_tans (wave-serial path), with the oracle's C decoder of it
    on one host thread."""
    import torch
    from bigsmall_amd.codecs import _refstreams
    from bigsmall_amd.codecs import bf16_chunked as bc
    from bigsmall_amd.device import ChunkBatch, ChunkJob, StatusWord, upload_bytes
    tensors = _c3_tensors()
    if args.c3_tensors:
        keep = set(args.c3_tensors.split(","))
        tensors = [(n, w) for n, w in tensors if n in keep]
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    res = {}
    # the format's default chunk (432 steps: sized for layer batches) gives one
    # 67M-element tensor 1,214 chunks, fewer than the 4,096 wavefront slots of
    # the GPU; 128 steps fill them (4,096 chunks) at a small ratio cost
    R = max(1, args.rotate)
    coders = [("rans_bsck", bc.CODER_RANS), ("tans_bsck", bc.CODER_TANS)]
    if args.rans_only:
        coders = coders[:1]
    for name, w in tensors:
        res[name] = {}
        for key, coder in coders:
            # the codecs' state counts (tANS: four states per wavefront lane);
            # fp8 tensors code byte pairs (one symbol per two bytes): half the
            # steps per chunk keep the chunk count, and so the GPU's fill, of
            # the bf16 tensors (4,096 chunks of 16,384 elements)
            lanes = args.lanes or (bc.TANS_LANES if coder == bc.CODER_TANS else bc.DEFAULT_LANES)
            steps = args.chunk_steps or max(16, (128 * 128 // lanes) // (2 if w.dtype == np.uint8 else 1))
            blob = bc.encode_array(w, steps=steps, lanes=lanes, coder=coder)
            inf = bc.info(blob)
            # R copies of the blob and of the output, decoded in turn: the working
            # set (R x up to 245 MB) is far beyond the 256 MB Infinity Cache
            d_blobs = [upload_bytes(blob, dev) for _ in range(R)]
            outs = [torch.empty(w.nbytes, dtype=torch.uint8, device=dev) for _ in range(R)]
            st = StatusWord(dev)
            batches = [ChunkBatch([ChunkJob(d.data_ptr(), len(blob), o.data_ptr(), w.size, inf.n_chunks,
                                            inf.plane_mode)], dev) for d, o in zip(d_blobs, outs)]
            it = iter(range(1 << 62))
            settle(lambda: batches[next(it) % R].launch(st, stream), args.settle_ms)
            for b in batches:
                b.launch(st, stream)
            ms = _timed(lambda: batches[next(it) % R].launch(st, stream), args.steps, stream)
            st.check(f"{name} {key}")
            src = torch.from_numpy(w.view(np.uint8).copy()).to(dev)
            for i, o in enumerate(outs):
                assert torch.equal(o, src), f"{name} {key}: copy {i} differs from the source"
            del src, outs, d_blobs, batches
            gbps = (len(blob) + w.nbytes) / (ms * 1e-3) / 1e9
            res[name][key] = {"codec": (bc.CODEC_BF16 if w.dtype == np.uint16 else bc.CODEC_FP8) if coder == 0 else
                              (bc.CODEC_BF16_TANS if w.dtype == np.uint16 else bc.CODEC_FP8_TANS),
                              "ms": round(ms, 4), "GBps": round(gbps, 2), "frac": round(gbps / HBM_PEAK_GBPS, 4),
                              "ratio_pct": round(100 * len(blob) / w.nbytes, 3), "plane_mode": inf.plane_mode,
                              "elem_bytes": inf.elem_bytes, "chunk_steps": steps, "lanes": lanes,
                              "distinct_copies": R}
            log(f"[c3] {name}: {key} mode {inf.plane_mode} {ms:.4f} ms, {gbps:.0f} GB/s "
                f"({100 * gbps / HBM_PEAK_GBPS:.1f} %), ratio {100 * len(blob) / w.nbytes:.2f} %")
    for name, (blob, cpu_gbps) in ({} if args.rans_only or args.engine_only else cpu_baseline_c3(tensors)).items():
        w = dict(tensors)[name]
        d_blob = upload_bytes(blob, dev)
        out = torch.empty(w.size, dtype=torch.int16, device=dev)
        st = StatusWord(dev)
        launch = _refstreams.RefLaunch(_refstreams.PARSERS["bf16_se_tans"](blob, w.size), d_blob.data_ptr(), dev,
                                       out.data_ptr())
        ms = _timed(lambda: launch.launch(out.data_ptr(), st.ptr, stream.cuda_stream), 1, stream)
        st.check(name)
        assert out.cpu().numpy().view(np.uint16).tobytes() == w.tobytes(), name
        gbps = (len(blob) + w.nbytes) / (ms * 1e-3) / 1e9
        res[name]["tans_reference_format"] = {"codec": "bf16_se_tans", "ms": round(ms, 1), "GBps": round(gbps, 4),
                                              "ratio_pct": round(100 * len(blob) / w.nbytes, 3),
                                              "cpu_baseline_GBps_1_thread": round(cpu_gbps, 4)}
        log(f"[c3] {name}: bf16_se_tans {ms:.0f} ms on GPU, oracle CPU {cpu_gbps:.3f} GB/s")
    head = res[next(iter(res))]["rans_bsck"]
    return {"metric": "decoded GB/s, 8192x8192 stress tensors (forced rANS and forced tANS on this engine's format; "
                      "the reference's bf16_se_tans beside them)",
            "value": head["GBps"], "unit": "GB/s", "n_gpus": 1, "ms_per_step": head["ms"], "higher_is_better": True,
            "dtype": "u32", "settle_ms": args.settle_ms,
            "data": "synthetic: Student-t df=3, half zeros, fp8 e4m3 + bf16 residual (seeded)",
            "host": host_cpu_info(), "config": {"workload": "c3_stress_8192sq", "elements_per_tensor": 8192 * 8192}, "tensors": res,
            "roofline": {"bound": "hbm", "achieved": head["GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": head["frac"]}}


def measure_h2d(dev, mib: int = 1024, reps: int = 5) -> float:
    """Host (pinned) -> device copy rate in the same run, bytes per second."""
    import torch
    n = mib << 20
    h = torch.empty(n, dtype=torch.uint8, pin_memory=True).fill_(1)
    d = torch.empty(n, dtype=torch.uint8, device=dev)
    d.copy_(h, non_blocking=True)
    ms = _timed(lambda: d.copy_(h, non_blocking=True), reps, torch.cuda.current_stream(dev))
    del h, d
    return n / (ms * 1e-3)


def run_streaming(args) -> dict:
    """BigSmallStreamingModel on a Llama-3-8B-shaped model cut to `--layers`
    layers (bf16, seeded N(0, 0.02) weights, 1 + N(0, 0.01) norms, untied
    embedding and lm_head 128256x4096): the container is written to a
    temporary file, and every forward pass (batch 1, 128 tokens) reads,
    copies and decodes each layer from it while the previous one runs. The
    floor is the PCIe transfer of a layer's compressed bytes at the
    host->device rate measured in the same run."""
    import shutil
    import tempfile
    import torch
    from transformers import LlamaConfig
    from bigsmall_amd import container
    from bigsmall_amd.encoder import compress
    from bigsmall_amd.streaming_inference import BigSmallStreamingModel
    n_layers = args.layers
    cfg = LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=n_layers,
                      num_attention_heads=32, num_key_value_heads=8, max_position_embeddings=2048,
                      tie_word_embeddings=False, attn_implementation="sdpa", torch_dtype="bfloat16")
    g = torch.Generator().manual_seed(0)

    def rnd(*shape):
        return (torch.randn(*shape, generator=g) * 0.02).bfloat16()

    def norm():
        return (1 + torch.randn(4096, generator=g) * 0.01).bfloat16()

    t0 = time.time()
    sd = {"model.embed_tokens.weight": rnd(128256, 4096), "lm_head.weight": rnd(128256, 4096), "model.norm.weight": norm()}
    for i in range(n_layers):
        for name, shape in LAYER:
            short = name.split("layers.0.")[1]
            sd[f"model.layers.{i}.{short}"] = norm() if "norm" in short else rnd(*shape)
    work = tempfile.mkdtemp(prefix="bs_stream_")
    try:
        path = os.path.join(work, "model.bs")
        compress(sd, path)
        cfg.save_pretrained(work)
        del sd
        log(f"[stream] {n_layers}-layer model written in {time.time() - t0:.1f}s ({os.path.getsize(path) / 1e9:.2f} GB)")
        hdr, _ = container.read_header(path)
        per_layer = sum(int(t["compressed_bytes"]) for t in hdr["tensors"] if t["name"].startswith("model.layers.0."))
        dev = torch.device("cuda", 0)
        h2d = measure_h2d(dev)
        ids = torch.randint(0, 128256, (1, 128), generator=torch.Generator().manual_seed(1)).cuda()
        res = {}
        for prefetch in (0, 1, 2):
            m = BigSmallStreamingModel.from_pretrained(path, device="cuda", prefetch=prefetch)
            m.forward(ids)
            torch.cuda.synchronize()
            ts = []
            for _ in range(args.steps):
                t1 = time.perf_counter()
                m.forward(ids)
                torch.cuda.synchronize()
                ts.append(time.perf_counter() - t1)
            m.close()
            res[prefetch] = sorted(ts)[len(ts) // 2]
            log(f"[stream] prefetch={prefetch}: {res[prefetch] * 1e3:.1f} ms per pass, "
                f"{res[prefetch] * 1e3 / n_layers:.2f} ms per layer")
        # the whole container into HBM with decoder.load (the same file)
        from bigsmall_amd import decoder
        file_bytes = os.path.getsize(path)
        loads = []
        for _ in range(3):
            t1 = time.perf_counter()
            sd = decoder.load(path, device="cuda")
            torch.cuda.synchronize()
            loads.append(time.perf_counter() - t1)
            del sd
        load_s = min(loads)
        log(f"[stream] decoder.load of the {file_bytes / 1e9:.2f} GB file: {load_s * 1e3:.1f} ms "
            f"({file_bytes / load_s / 1e9:.1f} GB/s of file)")
    finally:
        shutil.rmtree(work, ignore_errors=True)
    ms_layer = res[1] * 1e3 / n_layers
    floor_ms = per_layer / h2d * 1e3
    return {"metric": "ms per layer, BigSmallStreamingModel forward streaming an 8B-shaped model from a .bs file",
            "value": round(ms_layer, 3), "unit": "ms/layer", "n_gpus": 1, "steps": args.steps,
            "ms_per_step": round(res[1] * 1e3, 2), "higher_is_better": False, "dtype": "bf16",
            "data": "synthetic: seeded N(0,0.02) weights, 1+N(0,0.01) norms; batch 1, 128 tokens",
            "config": {"workload": "streaming_llama3_8b_shape", "layers": n_layers,
                       "compressed_bytes_per_layer": per_layer, "prefetch": 1},
            "prefetch0_ms_per_layer": round(res[0] * 1e3 / n_layers, 3),
            "prefetch2_ms_per_layer": round(res[2] * 1e3 / n_layers, 3),
            "decoder_load": {"file_bytes": file_bytes, "seconds": round(load_s, 4),
                             "file_GBps": round(file_bytes / load_s / 1e9, 2),
                             "frac_of_h2d": round(file_bytes / load_s / h2d, 4)},
            "pcie_floor": {"h2d_GBps": round(h2d / 1e9, 2), "ms_per_layer": round(floor_ms, 3),
                           "frac": round(floor_ms / ms_layer, 4)}}


def run_zstd(args) -> dict:
    """The reference's zstd-coded entries, decoded on the GPU from HBM:
    (a) the 65 RMSNorm weights of a Llama-3-8B-shaped model (4096 bf16 each,
    1 + N(0, 0.01)) as the reference's encoder writes them, special/lowcard
    with a level-19 zstd index frame (bigsmall/codecs/special.py:23-64), all in
    one bs_zstd_decode + bs_lut_expand launch pair; (b) one zstd_xor_delta frame
    of a 4096x4096 bf16 fine-tune that differs from its base in 1% of the
    elements (the reference's delta test shape, tests/test_delta.py:22-30),
    compressed at level 19. Beside each, libzstd (the format's reference
    implementation) on one host thread."""
    import torch
    from oracle import zstd_lib
    from bigsmall_amd.codecs.zstd_gpu import ZstdLaunch
    from bigsmall_amd.device import StatusWord, upload_bytes
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    rng = np.random.default_rng(6)

    def bf16(n, mean=0.0, std=0.02):
        x = (mean + rng.standard_normal(n) * std).astype(np.float32).view(np.uint32).astype(np.uint64)
        return ((x + 0x7FFF + ((x >> 16) & 1)) >> 16).astype(np.uint16)

    norms = [bf16(4096, 1.0, 0.01).tobytes() for _ in range(65)]
    blobs = [zstd_lib.encode_lowcard(r, 2)[0] for r in norms]
    t0 = time.perf_counter()
    for b, r in zip(blobs, norms):
        assert zstd_lib.decode_lowcard(b, len(r)) == r
    cpu_norms_ms = (time.perf_counter() - t0) * 1e3
    offs = np.cumsum([0] + [len(b) for b in blobs])
    d_blobs = upload_bytes(b"".join(blobs), dev)
    out = torch.empty(65 * 4096, dtype=torch.bfloat16, device=dev)
    z = ZstdLaunch(dev)
    for i, b in enumerate(blobs):
        z.add_lowcard(d_blobs.data_ptr() + int(offs[i]), b, out[i * 4096:].data_ptr(), 4096, 2)
    st = StatusWord(dev)
    z.launch(st, stream)
    torch.cuda.synchronize()
    st.check("norms")
    norms_ms = _timed(lambda: z.launch(st, stream), max(args.steps, 20), stream)
    st.check("norms timed")
    assert out.view(torch.int16).cpu().numpy().view(np.uint16).tobytes() == b"".join(norms)
    log(f"[zstd] 65 lowcard norms: {norms_ms * 1e3:.1f} us per launch pair on GPU; "
        f"libzstd + numpy on one host thread {cpu_norms_ms * 1e3:.0f} us")

    base = bf16(4096 * 4096)
    ft = base.copy()
    m = rng.random(base.size) < 0.01
    ft[m] ^= rng.integers(1, 8, int(m.sum())).astype(np.uint16)
    delta = (ft ^ base).tobytes()
    frame = zstd_lib.compress(delta, 19)
    t0 = time.perf_counter()
    assert zstd_lib.decompress(frame, len(delta)) == delta
    cpu_delta_ms = (time.perf_counter() - t0) * 1e3
    d_frame = upload_bytes(frame, dev)
    dst = torch.empty(len(delta), dtype=torch.uint8, device=dev)
    zd = ZstdLaunch(dev)
    zd.add_frame(d_frame.data_ptr(), len(frame), dst.data_ptr(), len(delta))
    zd.launch(st, stream)
    torch.cuda.synchronize()
    st.check("delta")
    delta_ms = _timed(lambda: zd.launch(st, stream), 2, stream)
    st.check("delta timed")
    assert dst.cpu().numpy().tobytes() == delta
    log(f"[zstd] 4096x4096 1% delta frame: {delta_ms:.1f} ms on GPU ({len(delta) / delta_ms / 1e6:.3f} GB/s); "
        f"libzstd one thread {cpu_delta_ms:.1f} ms")
    return {"metric": "microseconds to decode the 65 lowcard (zstd) RMSNorm entries of a Llama-3-8B-shaped model "
                      "on 1 MI355X",
            "value": round(norms_ms * 1e3, 2), "unit": "us", "n_gpus": 1, "ms_per_step": round(norms_ms, 4),
            "higher_is_better": False, "dtype": "u8",
            "data": "synthetic: seeded 1 + N(0, 0.01) bf16 norms; 1% XOR delta of N(0, 0.02) bf16; frames by libzstd",
            "host": host_cpu_info(),
            "config": {"workload": "zstd_lowcard_norms_65x4096", "frames": len(blobs),
                       "compressed_bytes": int(offs[-1]), "decoded_bytes": 65 * 4096 * 2},
            "roofline": {"bound": "latency (one workgroup per frame; zstd is sequential within a frame)",
                         "achieved": None, "peak": None, "unit": None, "frac": None},
            "delta_frame": {"decoded_bytes": len(delta), "frame_bytes": len(frame), "ms": round(delta_ms, 2),
                            "GBps": round(len(delta) / delta_ms / 1e6, 4),
                            "cpu_libzstd_ms_1_thread": round(cpu_delta_ms, 2)},
            "cpu_baseline": {"value": round(cpu_norms_ms * 1e3, 1), "unit": "us", "cores": 1, "kind": "reference",
                             "sample": "the same 65 lowcard blobs decoded by libzstd + numpy indexing "
                                       f"(libzstd {zstd_lib.version()})"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--settle-ms", type=float, default=50.0,
                    help="GPU workloads: run the workload untimed for this long before the warm-up steps, "
                         "so that the timed steps run at the clocks sustained load settles at (0: off)")
    ap.add_argument("--chunk-steps", type=int, default=None)
    ap.add_argument("--lanes", type=int, default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--two-streams", action="store_true",
                    help="layer workloads: also time the launches alternating between two streams")
    ap.add_argument("--rotate", type=int, default=6,
                    help="layer and c3 workloads: distinct compressed copies (and outputs) decoded in turn, so "
                         "the timed working set (6 x 725 MB for the layer) is far beyond the 256 MB Infinity Cache")
    ap.add_argument("--zero-fraction", type=float, default=0.0,
                    help="layer workload only: set this seeded share of every matrix's elements to +0.0 "
                         "(a pruned layer; such tensors take the compact plane mode)")
    ap.add_argument("--layers", type=int, default=8, help="streaming workload: decoder layers of the model")
    ap.add_argument("--workload", choices=["layer", "model", "kv", "refcodecs", "reflayer", "c3", "streaming", "zstd"],
                    default="layer",
                    help="layer (default: the headline line), model (full 8B-shaped model), kv (KV-cache "
                         "blocks), refcodecs (the reference's own formats on the C0 tensor), reflayer (the "
                         "headline layer in the reference's formats, one batched launch), c3 (stress "
                         "tensors), streaming (BigSmallStreamingModel forward from a .bs file), zstd (the "
                         "reference's zstd-coded entries: lowcard norms and a delta frame)")
    ap.add_argument("--c3-tensors", default="",
                    help="c3 workload: comma-separated subset of studentt,halfzero,fp8_e4m3,fp8_residual")
    ap.add_argument("--ref-codecs", default="",
                    help="reflayer workload: comma-separated subset of bf16_parallel_v1,bf16_se_tans")
    ap.add_argument("--ref-tables", choices=["auto", "lds", "scalar", "se-scalar", "mant-scalar"], default="auto",
                    help="refcodecs/reflayer/c3 workloads: where the reference formats' chains read their decode "
                         "tables (auto: the engine's choice; lds; scalar: SE and mantissa chains through the scalar "
                         "cache; se-scalar / mant-scalar: only those chains)")
    ap.add_argument("--coder", choices=["rans", "tans"], default="rans",
                    help="layer workload: the engine format's entropy coder (bf16_chunked_v1 or bf16_chunked_tans_v1)")
    ap.add_argument("--engine-only", action="store_true",
                    help="c3 workload: only this engine's format, rANS and tANS (skip the reference-format "
                         "bf16_se_tans decode and its CPU baseline)")
    ap.add_argument("--rans-only", action="store_true",
                    help="c3 workload: only this engine's format under rANS")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="only run device-to-device copies of this many MiB (calibrates FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--hbm-probe", action="store_true",
                    help="only measure 2 GiB read-only, write-only and copy streams (HBM rates by direction)")
    args = ap.parse_args()
    if args.ref_tables != "auto":
        from bigsmall_amd.codecs import _refstreams
        _refstreams.RefBatch.SE_SCALAR = args.ref_tables in ("scalar", "se-scalar")   # else False: every SE chain in LDS
        _refstreams.RefBatch.MANT_SCALAR = args.ref_tables in ("scalar", "mant-scalar")
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X; multi-GPU runs are not part of it (a model shards by "
              "tensor or layer for decoding, with no exchange between GPUs).", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.copy_probe_mb:
        copy_probe(args.copy_probe_mb)
        return
    if args.hbm_probe:
        print(json.dumps(hbm_probe(torch.device("cuda", 0))), flush=True)
        return
    if args.workload != "layer":
        run = {"model": run_model, "kv": run_kv, "refcodecs": run_refcodecs, "reflayer": run_reflayer, "c3": run_c3,
               "streaming": run_streaming, "zstd": run_zstd}[args.workload]
        print(json.dumps(run(args)), flush=True)
        return
    from bigsmall_amd.codecs import bf16_chunked as bc
    from bigsmall_amd.device import ChunkBatch, ChunkJob, StatusWord, upload_bytes

    tans = args.coder == "tans"
    # the tANS codec's geometry: four states per wavefront lane over half the steps
    steps = args.chunk_steps or (bc.tans_steps(bc.DEFAULT_STEPS) if tans else bc.DEFAULT_STEPS)
    lanes = args.lanes or (bc.TANS_LANES if tans else bc.DEFAULT_LANES)
    R = max(1, args.rotate)
    t0 = time.time()
    base_words = make_layer(0)
    workload = WORKLOAD
    if args.zero_fraction:
        base_words = zero_layer(base_words, args.zero_fraction)
        workload = f"{WORKLOAD}_{round(100 * args.zero_fraction)}pct_zeros"
    # R distinct layers (per-layer sign-flipped variants of the seeded draw; the
    # norms stay as drawn): step i decodes layer i mod R, so every step reads
    # and writes memory the previous R - 1 steps did not touch
    layers = [{name: (w if "norm" in name or r == 0 else _variants(w, r)) for name, w in base_words.items()}
              for r in range(R)]
    log(f"[bench] {R} layer(s) generated in {time.time() - t0:.1f}s")
    t0 = time.time()
    coder = bc.CODER_TANS if args.coder == "tans" else bc.CODER_RANS
    if coder == bc.CODER_TANS:
        workload += "_tans"
    blobs = [{name: bc.encode_array(w, steps=steps, lanes=lanes, coder=coder) for name, w in words.items()}
             for words in layers]
    log(f"[bench] encoded in {time.time() - t0:.1f}s")
    words = layers[0]
    n_total = sum(w.size for w in words.values())
    # copies of a layer without zeros compress to the same size; with zeros, the
    # sign flips turn some +0.0 into -0.0 and sizes differ slightly: the timed
    # launches' algorithmic bytes are then the mean over the copies they decode
    comp_sizes = [sum(len(b) for b in bl.values()) for bl in blobs]
    comp_total = round(sum(comp_sizes[i % R] for i in range(args.steps)) / max(1, args.steps))
    out_total = 2 * n_total
    algo_bytes = comp_total + out_total

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    # each compressed layer resident in HBM: one buffer per layer, blobs at 256-byte offsets
    d_comps, outs, batches = [], [], []
    for bl, lw in zip(blobs, layers):
        offs, pos = [], 0
        for name, _ in LAYER:
            pos = (pos + 255) & ~255
            offs.append(pos)
            pos += len(bl[name])
        host = np.zeros(pos, np.uint8)
        for (name, _), o in zip(LAYER, offs):
            host[o:o + len(bl[name])] = np.frombuffer(bl[name], np.uint8)
        d_comp = upload_bytes(host, dev)
        out = {name: torch.empty(lw[name].size, dtype=torch.bfloat16, device=dev) for name, _ in LAYER}
        jobs = [ChunkJob(d_comp.data_ptr() + o, len(bl[name]), out[name].data_ptr(), lw[name].size,
                         bc.info(bl[name]).n_chunks, bc.info(bl[name]).plane_mode) for (name, _), o in zip(LAYER, offs)]
        d_comps.append(d_comp)
        outs.append(out)
        batches.append(ChunkBatch(jobs, dev))
    status = StatusWord(dev)
    stream = torch.cuda.current_stream(dev)

    rot = iter(range(1 << 62))
    settled = settle(lambda: batches[next(rot) % R].launch(status, stream), args.settle_ms)
    for i in range(args.warmup):
        batches[i % R].launch(status, stream)
    torch.cuda.synchronize(dev)
    status.check("warmup")

    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    t_wall = time.perf_counter()
    ev0.record(stream)
    for i in range(args.steps):
        batches[i % R].launch(status, stream)
    ev1.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t_wall
    status.check("timed")
    ms_per = ev0.elapsed_time(ev1) / args.steps
    gbps = algo_bytes / (ms_per * 1e-3) / 1e9

    # With --two-streams: the same launches on two alternating streams, as the
    # engine's GroupDecoder issues consecutive layers (a launch's prologue runs
    # under the previous one's last workgroups). Reported beside the line;
    # `value` and the roofline stay the one-stream figure, one whole launch per
    # step, and the default run leaves it out so that a kernel trace of the
    # default command times non-overlapping launches only.
    ms_pipe = None
    if args.two_streams:
        alt = torch.cuda.Stream(dev)
        p0, p1, joined = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True), torch.cuda.Event()
        for i in range(max(2, args.warmup)):          # a stream's first launches set it up: untimed
            batches[i % R].launch(status, (stream, alt)[i % 2])
        torch.cuda.synchronize(dev)
        p0.record(stream)
        alt.wait_event(p0)
        for i in range(args.steps):
            batches[i % R].launch(status, (stream, alt)[i % 2])
        joined.record(alt)
        stream.wait_event(joined)
        p1.record(stream)
        torch.cuda.synchronize(dev)
        status.check("timed, two streams")
        ms_pipe = p0.elapsed_time(p1) / args.steps

    # verify bit-exactness (md5 per tensor, every layer copy) after timing; a
    # copy this run never decoded (fewer launches than copies) is decoded once first
    decoded = {i % R for i in range(args.warmup)} | {i % R for i in range(args.steps)}
    for i in range(R):
        if i not in decoded:
            batches[i].launch(status, stream)
    torch.cuda.synchronize(dev)
    status.check("untimed decode of the remaining layers")
    for out, lw in zip(outs, layers):
        for name, _ in LAYER:
            got = out[name].view(torch.int16).cpu().numpy().view(np.uint16)
            assert hashlib.md5(got.tobytes()).hexdigest() == hashlib.md5(lw[name].tobytes()).hexdigest(), name
    log(f"[bench] verified md5 of {len(LAYER)} tensors x {R} layers; {ms_per:.4f} ms/layer, {gbps:.1f} GB/s "
        f"(wall {wall:.3f}s)")
    del d_comps, outs, batches

    torch_copy_gbps = measure_copy(dev)
    kernel_copy_gbps = measure_copy_kernel(dev)
    copy_gbps = max(torch_copy_gbps, kernel_copy_gbps)
    log(f"[bench] device copy {torch_copy_gbps:.0f} GB/s (torch), {kernel_copy_gbps:.0f} GB/s (bs_copy_spans) "
        f"(read + write)")
    cpu = None if args.no_cpu_baseline else cpu_baseline(words, bsck_blobs=blobs[0])
    result = {
        "metric": "decoded bf16 GB/s on 1 MI355X (% of HBM roofline); ms per 8B-shaped layer",
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"ms": args.settle_ms, "launches": settled},
        "ms_per_step": round(ms_per, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic (seeded torch N(0,0.02) weights, 1+N(0,0.01) norms"
                + (f", {args.zero_fraction:g} of matrix elements zeroed" if args.zero_fraction else "")
                + "), encoded by the engine",
        "config": {
            "workload": workload,
            "tensors": len(LAYER), "elements": n_total, "decoded_bytes": out_total,
            "compressed_bytes": comp_total, "ratio_pct": round(100 * comp_total / out_total, 3),
            "codec": bc.CODEC_BF16_TANS if coder == bc.CODER_TANS else bc.CODEC_BF16, "chunk_steps": steps,
            "chunk_lanes": lanes, "launches_per_step": 1,
            "distinct_layers": R, "working_set_bytes": R * algo_bytes,
        },
        "ms_per_layer": round(ms_per, 5),
        "decoded_output_GBps": round(out_total / (ms_per * 1e-3) / 1e9, 2),
        "two_streams": None if ms_pipe is None else {
            "ms_per_layer": round(ms_pipe, 5), "GBps": round(algo_bytes / (ms_pipe * 1e-3) / 1e9, 2),
            "note": "the same launches alternating between two streams, as the engine decodes consecutive "
                    "layers: throughput of a sequence of layers, not one launch"},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": measured_traffic(workload),
                     "device_copy_GBps": round(copy_gbps, 1), "frac_of_device_copy": round(gbps / copy_gbps, 4),
                     "device_copy_note": f"2 GiB copy, the faster of torch's copy_ ({torch_copy_gbps:.0f} GB/s) "
                                         f"and bs_copy_spans ({kernel_copy_gbps:.0f} GB/s)"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
