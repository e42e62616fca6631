"""md5 verification of .bs containers (mirrors bigsmall/verify.py).

verify(src, source_safetensors=None) decodes every tensor on the GPU and
compares its md5 with the header's (encoder.py:375) or with the source file's
tensors (verify.py:14-51). verify_fast(src) checks structure without decoding
(verify.py:54-166): header parse, every blob inside the data section, every
codec one this engine decodes, tied refs resolvable.
"""
from __future__ import annotations

import hashlib
from pathlib import Path

from . import container
from .decoder import decompress


def verify(src: str | Path, source_safetensors: str | Path | None = None) -> bool:
    src = Path(src)
    header, _ = container.read_header(src)
    out = decompress(src)
    ok = True
    if source_safetensors is not None:
        import torch
        from safetensors import safe_open
        with safe_open(str(source_safetensors), framework="pt") as f:
            for name in f.keys():
                t = f.get_tensor(name)
                want = hashlib.md5(t.contiguous().view(torch.uint8).cpu().numpy().tobytes()).hexdigest()
                arr = out.get(name)
                if arr is None:
                    print(f"  MISSING {name}")
                    ok = False
                elif hashlib.md5(arr.tobytes()).hexdigest() != want:
                    print(f"  MISMATCH {name}")
                    ok = False
        return ok
    for t in header["tensors"]:
        got = hashlib.md5(out[t["name"]].tobytes()).hexdigest()
        if got != t["md5"]:
            print(f"  MISMATCH {t['name']} hdr={t['md5']} dec={got}")
            ok = False
    return ok


def verify_fast(src: str | Path, verbose: bool = False) -> tuple[bool, list[str]]:
    from .engine import check_supported
    from .exceptions import BigSmallVersionError
    src = Path(src)
    problems: list[str] = []
    try:
        header, data_offset = container.read_header(src)
    except Exception as e:  # noqa: BLE001 - report, do not raise
        return False, [f"header: {e}"]
    data_size = src.stat().st_size - data_offset
    names = {t["name"] for t in header.get("tensors", [])}
    for t in header.get("tensors", []):
        off, nb = int(t.get("offset", -1)), int(t.get("compressed_bytes", -1))
        if off < 0 or nb < 0 or off + nb > data_size:
            problems.append(f"{t['name']}: blob [{off}, +{nb}) outside data section of {data_size} bytes")
        try:
            check_supported(t)
        except BigSmallVersionError:
            problems.append(f"{t['name']}: codec {t['codec']!r} is not decodable by this engine")
        if t["codec"] == "tied_ref" and (t.get("extra") or {}).get("tied_to") not in names:
            problems.append(f"{t['name']}: tied_ref master missing")
    if header.get("tensor_count") != len(header.get("tensors", [])):
        problems.append("tensor_count does not match the tensor list")
    if verbose and not problems:
        print(f"  tensors: {len(header['tensors'])}  data section: {data_size} bytes")
    return not problems, problems
