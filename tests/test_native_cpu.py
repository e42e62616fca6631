"""CPU checks of the native library (no GPU needed):

- libbigsmall_hip.so loads and exports every function include/bigsmall_hip.h declares;
- the host encoder of the GPU-native format (bf16_chunked_v1) round-trips
  through the oracle's independent CPU decoder, for every plane mode, both
  state-group widths and awkward sizes;
- planted mistakes in a blob are caught by the oracle decoder.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import oracle

ROOT = Path(__file__).resolve().parents[1]


def _bf16(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _declared_functions() -> list[str]:
    names = []
    for hdr in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", hdr.read_text(), flags=re.S)
        names += re.findall(r"^\s*(?:int|uint32_t|uint64_t)\s+(bs_\w+)\s*\(", text, flags=re.M)
    return names


def test_library_exports_every_declared_symbol():
    from bigsmall_amd import _native
    L = _native.lib()
    names = _declared_functions()
    assert len(names) >= 7
    for n in names:
        assert hasattr(L, n), f"{n} declared in include/ but not exported"
        assert n in _native.SIGNATURES, f"{n} has no ctypes signature"
    assert L.bs_version() >= 100


@pytest.fixture(scope="module", autouse=True)
def _oracle():
    oracle.build()


@pytest.mark.parametrize("lanes", [64, 128, 256])
@pytest.mark.parametrize("mode", [-1, 1, 2])
@pytest.mark.parametrize("n", [1, 2, 63, 64, 129, 1000, 65536 + 7, 300_000])
def test_encoder_roundtrip_via_oracle(n, mode, lanes):
    from bigsmall_amd.codecs import bf16_chunked as bc
    rng = np.random.default_rng(n * 7 + mode)
    w = _bf16(rng.standard_normal(n) * 0.02)
    if n > 100:
        w[rng.permutation(n)[: n // 3]] = 0
    blob = bc.encode_array(w, mode=mode, lanes=lanes, steps=64)
    assert oracle.chunk_decode(blob, n) == w.tobytes()
    inf = bc.info(blob)
    assert inf.n == n and inf.lanes == lanes and (mode < 0 or inf.plane_mode == mode)


def test_exact_and_byte_modes_via_oracle():
    from bigsmall_amd.codecs import bf16_chunked as bc
    rng = np.random.default_rng(1)
    norm = _bf16(1.0 + rng.standard_normal(4096) * 0.01)
    blob = bc.encode_array(norm)
    assert bc.info(blob).plane_mode == 0 and len(blob) < 0.3 * norm.nbytes
    assert oracle.chunk_decode(blob, norm.size) == norm.tobytes()
    b8 = rng.integers(0, 256, 70_001).astype(np.uint8)
    blob = bc.encode_array(b8)
    assert oracle.chunk_decode(blob, b8.size, 1) == b8.tobytes()
    allw = rng.integers(0, 65536, 50_000).astype(np.uint16)
    blob = bc.encode_array(allw)
    assert oracle.chunk_decode(blob, allw.size) == allw.tobytes()


def test_ratio_close_to_reference_codecs():
    """The GPU-native layout costs < 1.5 pp of ratio against the reference's
    bf16_se_tans on Gaussian weights (same data, both measured here)."""
    from bigsmall_amd.codecs import bf16_chunked as bc
    rng = np.random.default_rng(2)
    w = _bf16(rng.standard_normal(1 << 21) * 0.02)
    mine = len(bc.encode_array(w))
    ref = len(oracle.tans_encode(w))
    assert (mine - ref) / w.nbytes * 100 < 1.5


def test_planted_corruption_is_caught():
    from bigsmall_amd.codecs import bf16_chunked as bc
    rng = np.random.default_rng(3)
    w = _bf16(rng.standard_normal(100_000) * 0.02)
    blob = bytearray(bc.encode_array(w))
    ctab = (32 + 4 * int.from_bytes(blob[22:24], "little") + 15) & ~15
    off = int.from_bytes(blob[ctab:ctab + 8], "little")
    lanes = int.from_bytes(blob[20:22], "little")
    blob[off + 4 * lanes + 6] ^= 0x33          # a renorm word
    try:
        out = oracle.chunk_decode(bytes(blob), w.size)
        assert out != w.tobytes()
    except oracle.OracleError:
        pass
    bad = bytearray(bc.encode_array(w))
    bad[32 + 2] ^= 0x01                         # a frequency: sum != 4096
    with pytest.raises(oracle.OracleError):
        oracle.chunk_decode(bytes(bad), w.size)


@pytest.mark.parametrize("field,value", [("magic", b"BSCX"), ("version", 4), ("version", 1), ("elem_bytes", 3),
                                         ("plane_mode", 3), ("plane_mode", 4), ("prec", 11), ("lanes", 96),
                                         ("steps", 24), ("n_syms", 0), ("n_chunks", 7), ("coder", 3),
                                         ("truncated", None)])
def test_malformed_header_raises_value_error(field, value):
    """bs_chunk_inspect (host code) rejects every malformed header field, and
    the codec turns that into ValueError, as the reference does for bad magic
    or counts (bigsmall/codecs/bf16_parallel.py:153-163)."""
    import struct
    from bigsmall_amd.codecs import bf16_chunked as bc
    w = _bf16(np.random.default_rng(4).standard_normal(50_000) * 0.02)
    head = bytearray(bc.encode_array(w)[:32])
    assert bc.info(bytes(head)).n == w.size
    offs = {"version": (4, "<B"), "elem_bytes": (5, "<B"), "plane_mode": (6, "<B"), "prec": (7, "<B"),
            "lanes": (20, "<H"), "steps": (16, "<I"), "n_syms": (22, "<H"), "n_chunks": (24, "<I"),
            "coder": (28, "<I")}
    if field == "magic":
        head[0:4] = value
    elif field == "truncated":
        head = head[:31]
    else:
        o, fmt = offs[field]
        struct.pack_into(fmt, head, o, value)
    with pytest.raises(ValueError):
        bc.info(bytes(head))


def test_chunk_size_is_capped_at_2_pow_24_elements():
    """A chunk holds at most 2^24 elements (lanes x steps), so byte offsets
    inside a chunk fit 32 bits: the host header check and both encoders'
    argument checks refuse one more step block, and accept the cap itself."""
    import ctypes
    import struct
    from bigsmall_amd import _native
    from bigsmall_amd.codecs import bf16_chunked as bc
    w = _bf16(np.random.default_rng(5).standard_normal(50_000) * 0.02)
    head = bytearray(bc.encode_array(w)[:32])
    assert struct.unpack_from("<I", head, 24)[0] == 1          # one chunk either way
    struct.pack_into("<I", head, 16, (1 << 24) // 128)          # 128 x 131072 = 2^24: accepted
    assert bc.info(bytes(head)).steps == 131072
    struct.pack_into("<I", head, 16, (1 << 24) // 128 + 16)     # one step block more: refused
    with pytest.raises(ValueError):
        bc.info(bytes(head))
    L = _native.lib()
    bound = ctypes.c_uint64()
    assert L.bs_chunk_encode_bound(1000, 2, 128, 131072, ctypes.byref(bound)) == 0
    assert L.bs_chunk_encode_bound(1000, 2, 128, 131072 + 16, ctypes.byref(bound)) != 0
    assert L.bs_chunk_encode_bound(1000, 2, 256, 65536 + 16, ctypes.byref(bound)) != 0


def test_invariant_divisor_multiply_shift_is_exact():
    """The GPU encoder divides a 32-bit state by a symbol frequency f (1..4096)
    with Granlund and Montgomery's multiply-shift (PLDI 1994, Figure 4.1;
    div_constants / div_by_freq in csrc/bsck_encode_gpu.hip, restated here):
    it must equal x // f for every divisor, on random dividends and on every
    quotient boundary near the ends of the 32-bit range."""
    rng = np.random.default_rng(9)
    f = np.arange(1, 4097, dtype=np.uint64)
    l = np.array([0 if v == 1 else int(v - 1).bit_length() for v in f], dtype=np.uint64)
    m = ((np.uint64(1) << np.uint64(32)) * ((np.uint64(1) << l) - f)) // f + np.uint64(1)
    assert int(m.max()) < (1 << 32)
    s1 = np.minimum(l, 1)
    s2 = np.where(l > 0, l - 1, 0).astype(np.uint64)
    rand = rng.integers(0, 1 << 32, size=(4096, 64), dtype=np.uint64)
    q_top = (np.uint64((1 << 32) - 1) // f)[:, None]
    edges = np.concatenate([f[:, None] * q_top - np.uint64(1), f[:, None] * q_top, np.full((4096, 1), (1 << 32) - 1, np.uint64),
                            np.zeros((4096, 1), np.uint64), f[:, None] - np.uint64(1), f[:, None], (f[:, None] << np.uint64(20)) - np.uint64(1)],
                           axis=1) & np.uint64(0xFFFFFFFF)
    x = np.concatenate([rand, edges], axis=1)
    t = (m[:, None] * x) >> np.uint64(32)
    q = (t + ((x - t) >> s1[:, None])) >> s2[:, None]
    assert np.array_equal(q, x // f[:, None])


def test_struct_layouts_match_the_header(tmp_path):
    """Every struct the C-ABI takes has a host-side mirror (numpy dtype or
    ctypes Structure) that the library reads as raw bytes; each field's offset
    and size must equal the C compiler's layout of include/bigsmall_hip.h."""
    import shutil
    import subprocess

    import numpy as np
    from bigsmall_amd import _native
    from bigsmall_amd.codecs import _refstreams, bf16_chunked, zstd_gpu
    from bigsmall_amd.device import TASK_DTYPE
    if shutil.which("gcc") is None:
        pytest.skip("needs gcc")
    structs = {
        "bs_chunk_info": (["n", "n_chunks", "steps", "lanes", "n_syms", "elem_bytes", "plane_mode", "coder"],
                          [(f[0], getattr(_native.BsChunkInfo, f[0]).offset, ctypes.sizeof(f[1]))
                           for f in _native.BsChunkInfo._fields_]),
        "bs_chunk_task": (["blob", "blob_bytes", "out", "n", "wg_begin", "n_chunks"], TASK_DTYPE),
        "bs_encode_task": (["src", "n", "dst", "cap", "chunk_begin", "n_chunks", "seg_len", "seg_stride"],
                           bf16_chunked.ENCODE_TASK_DTYPE),
        "bs_span": (["src", "dst", "len"], bf16_chunked.SPAN_DTYPE),
        "bs_se_stream": (["words", "x0", "n_words", "tail", "n", "first", "stride", "reserved"],
                         _refstreams.SE_STREAM_DTYPE),
        "bs_mant_bucket": (["words", "x0", "n_words", "tail", "n", "perm_begin", "table", "reserved"],
                           _refstreams.MANT_BUCKET_DTYPE),
        "bs_ref_task": (["streams", "se_table", "bstart", "buckets", "mant_tables", "out", "n_out", "work_offset",
                         "n_streams", "n_buckets", "n_tables", "se_group_begin", "tile_begin", "stream_begin",
                         "mant_group_begin", "flags"],
                        _refstreams.REF_TASK_DTYPE),
        "bs_zstd_task": (["src", "src_len", "dst", "dst_len", "xor_src"], zstd_gpu.ZSTD_TASK_DTYPE),
        "bs_lut_task": (["idx", "lut", "out", "n", "n_lut", "item_bytes"], zstd_gpu.LUT_TASK_DTYPE),
    }
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "bigsmall_hip.h"', "int main(void) {"]
    for st, (fields, _) in structs.items():
        lines.append(f'  printf("{st} sizeof %zu\\n", sizeof({st}));')
        for f in fields:
            lines.append(f'  printf("{st} {f} %zu %zu\\n", offsetof({st}, {f}), sizeof((({st}*)0)->{f}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    inc = Path(__file__).resolve().parents[1] / "include"
    subprocess.run(["gcc", "-I", str(inc), str(src), "-o", str(exe)], check=True, capture_output=True)
    got: dict = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        parts = line.split()
        if parts[1] == "sizeof":
            got[(parts[0], "sizeof")] = int(parts[2])
        else:
            got[(parts[0], parts[1])] = (int(parts[2]), int(parts[3]))
    for st, (fields, mirror) in structs.items():
        if isinstance(mirror, np.dtype):
            assert mirror.itemsize == got[(st, "sizeof")], st
            py = [(name, mirror.fields[name][1], mirror.fields[name][0].itemsize) for name in mirror.names]
        else:
            assert ctypes.sizeof(_native.BsChunkInfo) == got[(st, "sizeof")], st
            py = mirror
        assert len(py) == len(fields), st
        for (name, off, size), f in zip(py, fields):
            assert (off, size) == got[(st, f)], (st, f, name)
