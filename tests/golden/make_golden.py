"""Write golden input/output vectors for the rANS-family codecs.

Runs ONLY in the build container, where the reference checkout lives at
/root/reference. It loads the reference's pure-Python codec modules by file
path (bigsmall/codecs/rans.py, bf16_parallel.py, numba_rans.py, bf16_tans.py,
single_kernel.py) under a synthetic ``bigsmall.codecs`` package so the
package ``__init__`` files (which import the absent ``constriction`` /
``zstandard`` / ``blosc2``) are never executed. The five modules need only
numpy plus the bf16 bit-layout constants that ``bigsmall/codecs/bf16.py:25-30``
defines; those constants are provided here by value. numba is absent, so
``numba_rans.py:26-37`` and ``single_kernel.py:26-36`` run their pure-Python
fallbacks (same arithmetic, slower).

Output: tests/golden/ref_vectors.npz — data only (uint8/uint16/int64/uint32
arrays): inputs and the reference's outputs. Nothing of the reference's source
is stored. Sizes are kept small because the fallbacks run ~10 us/symbol.

With --routing it instead writes tests/golden/routing_vectors.npz: the
reference's own `tensor_analysis.analyze_tensors` (bigsmall/tensor_analysis.py,
which imports only hashlib and numpy, loaded by path the same way) run over a
list of tensors built to sit on each side of its thresholds; stored are the
tensors (raw bytes, shape, item size, dtype string, name) and the decisions
(kind and tied_to), as data.

Usage:  python tests/golden/make_golden.py [--routing]
"""
from __future__ import annotations

import importlib.util
import sys
import time
import types
from pathlib import Path

import numpy as np

REF = Path("/root/reference/bigsmall/codecs")
OUT = Path(__file__).resolve().parent / "ref_vectors.npz"
ROUTING_OUT = Path(__file__).resolve().parent / "routing_vectors.npz"


def _load_reference_codecs():
    pkg = types.ModuleType("bigsmall")
    pkg.__path__ = []
    sub = types.ModuleType("bigsmall.codecs")
    sub.__path__ = []
    consts = types.ModuleType("bigsmall.codecs.bf16")
    # bit layout of bf16 (bigsmall/codecs/bf16.py:25-30)
    consts.SIGN_SHIFT, consts.EXP_SHIFT, consts.EXP_MASK, consts.MANT_MASK = 15, 7, 0xFF, 0x7F
    consts.SE_ALPHABET, consts.MANT_ALPHABET = 512, 128
    sys.modules.update({"bigsmall": pkg, "bigsmall.codecs": sub, "bigsmall.codecs.bf16": consts})
    mods = {}
    for name in ["rans", "bf16_parallel", "numba_rans", "bf16_tans", "single_kernel"]:
        spec = importlib.util.spec_from_file_location(f"bigsmall.codecs.{name}", REF / f"{name}.py")
        mod = importlib.util.module_from_spec(spec)
        sys.modules[spec.name] = mod
        spec.loader.exec_module(mod)
        mods[name] = mod
    return mods


def _bf16_words(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit pattern with round-to-nearest-even (torch's .to(bfloat16))."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def _inputs() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(20240601)
    edge = np.array([0x7FC0, 0x7F80, 0xFF80, 0x0000, 0x8000, 0x0001, 0x0080, 0x3F80], np.uint16)
    gauss_small = _bf16_words(rng.standard_normal(4096) * 0.02)
    cases = {
        # edge words + normals (mirrors tests/test_bf16_parallel.py:39-62 in the reference)
        "edge": np.concatenate([edge, gauss_small]),
        "gauss": _bf16_words(rng.standard_normal(65536) * 0.02),
        "tiny": _bf16_words(rng.standard_normal(5) * 0.02),
        "zeros": np.zeros(1000, np.uint16),
        "halfzero": None,
        "studentt": _bf16_words(rng.standard_t(3, 32768) * 0.02 / np.sqrt(3.0)),
        "norm": _bf16_words(1.0 + rng.standard_normal(4096) * 0.01),
        "one": np.array([0x3F80], np.uint16),
    }
    hz = _bf16_words(rng.standard_normal(32768) * 0.02)
    hz[rng.permutation(32768)[:16384]] = 0
    cases["halfzero"] = hz
    return cases


def _count_vectors(rng) -> list[tuple[np.ndarray, int]]:
    vecs = []
    vecs.append((np.zeros(512, np.int64), 4096))                      # n_nz == 0
    c = np.zeros(128, np.int64); c[5] = 77; vecs.append((c, 1024))    # single symbol
    vecs.append((rng.integers(0, 1000, 512).astype(np.int64), 4096))  # dense random
    c = np.zeros(512, np.int64); c[rng.choice(512, 40, replace=False)] = rng.integers(1, 5, 40)
    vecs.append((c, 4096))                                            # many ties
    c = np.zeros(128, np.int64); c[:100] = 1; c[100] = 10**9          # diff < 0 (min-1 bumps)
    vecs.append((c, 1024))
    c = np.zeros(512, np.int64); c[:300] = 1; c[300] = 5 * 10**6; c[301] = 7
    vecs.append((c, 4096))
    c = rng.integers(0, 3, 128).astype(np.int64) * 1000 + 1           # equal-value ties
    vecs.append((c, 1024))
    g = _bf16_words(rng.standard_normal(200000) * 0.02)
    se = ((g >> 15) << 8 | ((g >> 7) & 0xFF)).astype(np.int64)
    vecs.append((np.bincount(se, minlength=512).astype(np.int64), 4096))
    return vecs


def main() -> None:
    t0 = time.time()
    m = _load_reference_codecs()
    rans, par, tans, sk = m["rans"], m["bf16_parallel"], m["bf16_tans"], m["single_kernel"]
    rng = np.random.default_rng(7)
    out: dict[str, np.ndarray] = {}

    # rans.py:34-92 and single_kernel.py:53-110 quantisers
    for i, (c, M) in enumerate(_count_vectors(rng)):
        out[f"q{i}_counts"] = c
        out[f"q{i}_M"] = np.array([M], np.int64)
        try:
            out[f"q{i}_ref"] = rans.quantise_frequencies(c, M).astype(np.uint32)
        except RuntimeError:
            # rans.py:88-90: the reference gives up; the oracle must too
            out[f"q{i}_ref_raises"] = np.array([1], np.int64)
        q = np.zeros(len(c), np.uint32)
        sk._quantise_inplace(c.copy(), np.int64(M), q)
        out[f"q{i}_sk"] = q

    # rans.py:115-207 stream encode/decode
    for i, (alpha, M, n) in enumerate([(512, 4096, 3000), (128, 1024, 2000), (4, 1024, 500)]):
        p = rng.dirichlet(np.ones(alpha) * 0.3)
        syms = rng.choice(alpha, n, p=p).astype(np.int32)
        freqs = rans.quantise_frequencies(np.bincount(syms, minlength=alpha), M)
        blob = rans.encode_stream(syms, freqs, M)
        dec = rans.decode_stream(blob, n, freqs, rans.build_slot_to_symbol(freqs, M), M)
        assert np.array_equal(dec.astype(np.int32), syms)
        out[f"s{i}_syms"], out[f"s{i}_freqs"] = syms, freqs.astype(np.uint32)
        out[f"s{i}_M"] = np.array([M], np.int64)
        out[f"s{i}_blob"] = np.frombuffer(blob, np.uint8)

    # codec blobs
    cases = _inputs()
    for name, words in cases.items():
        raw = words.astype("<u2").tobytes()
        out[f"in_{name}"] = words
        for ns in ([1, 3, 32, 128] if name in ("edge", "tiny") else [64]):
            blob, _ = par.encode(raw, n_streams=ns)
            assert par.decode(blob, {}, len(words)) == raw
            out[f"par1_{name}_N{ns}"] = np.frombuffer(blob, np.uint8)
        if len(words) <= 40000 or name == "gauss":
            blob, _ = tans.encode(raw)
            assert tans.decode(blob, {}, len(words)) == raw
            out[f"tans_{name}"] = np.frombuffer(blob, np.uint8)
            # single_kernel.py's decoder is not run here: without numba, under
            # numpy 2, its `in_buf[pos] | (in_buf[pos + 1] << 8)` field reads
            # wrap in uint8 (single_kernel.py:442-443), so only its encoder
            # (pure integer/uint64 arithmetic) is recorded. The oracle's
            # decoder is checked against these blobs by losslessness.
            blob, _ = sk.encode(raw)
            out[f"sk_{name}"] = np.frombuffer(blob, np.uint8)
        print(f"{name}: done ({time.time() - t0:.1f}s)", flush=True)

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays) in {time.time() - t0:.1f}s")


def _routing_tensors() -> list[dict]:
    """Tensors on both sides of analyze_tensors' thresholds: 16 / 17 distinct
    values, 255 / 256 bytes, a first sample of 4096 elements with few values
    followed by many, ties of equal bytes under another dtype, another shape
    and below 1024 bytes, a tie whose master is lowcard, row-correlated 2-D
    tensors with 16 and 15 rows, item sizes 1, 2, 4 and 8, an empty tensor."""
    rng = np.random.default_rng(31)

    def t(name, arr, dtype, shape=None):
        a = np.ascontiguousarray(arr)
        return {"name": name, "shape": list(shape if shape is not None else a.shape), "dtype": dtype,
                "item_bytes": a.dtype.itemsize, "raw": a.tobytes()}

    norm = lambda: _bf16_words(1.0 + rng.standard_normal(4096) * 0.01)       # C1 RMSNorm vectors
    gauss = _bf16_words(rng.standard_normal(64 * 512) * 0.02).reshape(64, 512)
    rows = np.arange(128)[:, None] / 20.0 + np.arange(128)[None, :] / 7.0
    smooth = _bf16_words(1.0 + 0.1 * np.sin(rows))                          # position-embedding-like
    rows15 = np.arange(15)[:, None] / 20.0 + np.arange(1024)[None, :] / 7.0
    n0, n1 = norm(), norm()
    late = np.concatenate([np.zeros(4096, np.uint16), rng.integers(0, 65536, 4096).astype(np.uint16)])
    return [
        t("model.layers.0.input_layernorm.weight", n0, "bfloat16"),
        t("model.layers.0.post_attention_layernorm.weight", n1, "bfloat16"),
        t("sixteen_values", rng.choice(rng.integers(0, 65536, 16).astype(np.uint16), 2048), "bfloat16"),
        t("seventeen_values", np.resize(np.arange(17, dtype=np.uint16) * 3, 2048), "bfloat16"),
        t("lowcard_255_bytes", rng.integers(0, 3, 255).astype(np.uint8), "uint8"),
        t("lowcard_256_bytes", rng.integers(0, 3, 256).astype(np.uint8), "uint8"),
        t("few_then_many", late, "bfloat16"),
        t("embed", gauss, "bfloat16"),
        t("embed_as_fp16", gauss, "float16"),                                 # same bytes, other dtype
        t("embed_other_shape", gauss, "bfloat16", shape=[128, 256]),
        t("small_a", _bf16_words(rng.standard_normal(400) * 0.02), "bfloat16"),
        t("wpe", smooth, "bfloat16"),
        t("wpe_15_rows", _bf16_words(1.0 + 0.1 * np.sin(rows15)), "bfloat16"),
        t("fp32_three_values", rng.choice(np.array([0.0, 1.0, -1.0], np.float32), 1024), "float32"),
        t("int64_counts", rng.integers(0, 5, 512).astype(np.int64), "int64"),
        t("norm_copy", n0, "bfloat16"),                                       # tied to a lowcard master
        t("zeros", np.zeros(4096, np.uint16), "bfloat16"),
        t("empty", np.zeros(0, np.uint16), "bfloat16"),
    ]


def routing_main() -> None:
    import json
    spec = importlib.util.spec_from_file_location("bigsmall.tensor_analysis", REF.parent / "tensor_analysis.py")
    ta = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(ta)
    tensors = _routing_tensors()
    # small_a appears twice: equal bytes below 1024, which are never tied
    tensors.insert(11, dict(tensors[10], name="small_b"))
    decisions, tied_map = ta.analyze_tensors(tensors)
    out = {f"raw{i}": np.frombuffer(tt["raw"], np.uint8) for i, tt in enumerate(tensors)}
    meta = [{k: tt[k] for k in ("name", "shape", "dtype", "item_bytes")} for tt in tensors]
    out["meta"] = np.array(json.dumps(meta))
    out["decisions"] = np.array(json.dumps(decisions))
    out["tied_map"] = np.array(json.dumps({str(k): v for k, v in tied_map.items()}))
    np.savez_compressed(ROUTING_OUT, **out)
    for m, d in zip(meta, decisions):
        print(f"{m['name']:48s} {d['kind']:10s} {d['tied_to']}")
    print(f"wrote {ROUTING_OUT} ({ROUTING_OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    if "--routing" in sys.argv[1:]:
        routing_main()
    else:
        main()
