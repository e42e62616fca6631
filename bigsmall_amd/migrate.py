"""BigSmall `migrate`: re-encode a .bs file with the current codec selection.

The reference's `bigsmall/migrate.py:1-210`: the same function, arguments,
result keys and rules.
  * Entries whose codec is `tied_ref`, `raw`, `special` or `zstd_xor_delta`
    are kept as they are (migrate.py:41-43).
  * Every other entry is decoded (on the GPU, through decoder._decode_blob) and
    offered to codec_registry.auto_select_codec. The new blob replaces the old
    one only when it is smaller; an entry that does not decode here (a
    constriction codec) or that no candidate encodes is kept.
  * Delta containers are not migrated (migrate.py:94-108).
  * The output is version 2 when any entry uses a version-2 codec
    (formats.V2_CODECS, which holds this engine's GPU formats), else version 1,
    as encoder.compress stamps it.

So a container the reference wrote migrates into this engine's GPU formats
wherever they are smaller.

Layout: blobs back to back, as the reference writes them, except that a blob
re-encoded into a BSCK codec starts on a 16-byte boundary (the kernels read it
with 16-byte loads; an unaligned one costs the loader a device copy). Such a
blob is taken only when its padding plus its length is below the original's
length, so the migrated file is never larger than the original.
"""
from __future__ import annotations

import shutil
from pathlib import Path

from . import codec_registry, container, formats
from .decoder import _decode_blob
from .engine import BSCK_CODECS

# payloadless, or already the best codec for their data pattern (migrate.py:41-43)
_KEEP_AS_IS_CODECS = frozenset({"tied_ref", "raw", "special", "zstd_xor_delta"})
_BSCK_ALIGN = 16


def _fmt_for_dtype(dtype_str: str) -> str:
    """The entry's BigSmall format key; "raw" (generic candidates) for a
    dtype without one (migrate.py:46-55)."""
    try:
        return formats.detect_format_from_dtype(dtype_str)
    except ValueError:
        return "raw"


def migrate(src: str | Path, dry_run: bool = False, backup: bool = True) -> dict:
    """Re-encode `src` in place (migrate.py:58-210); `dry_run` computes the
    savings and writes nothing, `backup` first copies the original to
    `<src>.bak`. Returns tensors_total, tensors_migrated, bytes_before,
    bytes_after (blob bytes), savings_pct, file_size_before, file_size_after,
    format_version, dry_run and codec_changes ({"old->new": count}); a delta
    container also gets skipped_reason. Errors from container.read_header
    (not a .bs file, an unsupported version) propagate."""
    src = Path(src)
    header, data_offset = container.read_header(src)
    file_size_before = src.stat().st_size
    if header.get("model_type") == "delta":
        section = file_size_before - data_offset
        return {"tensors_total": header.get("tensor_count", 0), "tensors_migrated": 0,
                "bytes_before": section, "bytes_after": section, "savings_pct": 0.0,
                "file_size_before": file_size_before, "file_size_after": file_size_before,
                "format_version": header.get("_format_version", formats.BS_FORMAT_VERSION_V1),
                "dry_run": dry_run, "codec_changes": {}, "skipped_reason": "delta_container_not_migrated"}
    with open(src, "rb") as f:
        f.seek(data_offset)
        data = f.read()

    parts: list[bytes] = []
    offset = bytes_before = bytes_after = migrated = 0
    changes: dict[str, int] = {}
    entries: list[dict] = []
    for t in header["tensors"]:
        blob = data[t["offset"]:t["offset"] + t["compressed_bytes"]]
        out, codec, extras, pad = blob, t["codec"], t.get("extra"), 0
        if codec not in _KEEP_AS_IS_CODECS:
            try:
                raw = _decode_blob(t, blob)
            except Exception:                      # not decodable here: kept as it is
                raw = None
            if raw:
                try:
                    cand, cand_codec, cand_extras = codec_registry.auto_select_codec(
                        raw, fmt=_fmt_for_dtype(t["dtype"]), dtype=t["dtype"], tensor_name=t.get("name", ""),
                        shape=tuple(t.get("shape") or ()))
                except Exception:
                    cand = None
                if cand is not None:
                    cand_pad = (-offset) % _BSCK_ALIGN if cand_codec in BSCK_CODECS else 0
                    if cand_pad + len(cand) < len(blob):
                        changes[f"{codec}->{cand_codec}"] = changes.get(f"{codec}->{cand_codec}", 0) + 1
                        out, codec, extras, pad = cand, cand_codec, cand_extras or {}, cand_pad
                        migrated += 1
        bytes_before += len(blob)
        bytes_after += len(out)
        if pad:
            parts.append(b"\x00" * pad)
            offset += pad
        entry = {k: v for k, v in t.items() if k != "_format_version"}
        entry.update(codec=codec, compressed_bytes=len(out), offset=offset, extra=extras or None)
        entries.append(entry)
        parts.append(out)
        offset += len(out)

    stats: dict[str, int] = {}
    for e in entries:
        stats[e["codec"]] = stats.get(e["codec"], 0) + 1
    out_header = {k: v for k, v in header.items() if not k.startswith("_") and k not in ("tensors", "codec_stats")}
    out_header.update(tensors=entries, tensor_count=len(entries), codec_stats=stats)
    version = formats.BS_FORMAT_VERSION_V2 if any(e["codec"] in formats.V2_CODECS for e in entries) \
        else formats.BS_FORMAT_VERSION_V1

    file_size_after = file_size_before
    if not dry_run:
        if backup:
            shutil.copy2(src, src.with_suffix(src.suffix + ".bak"))
        tmp = src.with_suffix(src.suffix + ".tmp")
        container.write_container(tmp, out_header, b"".join(parts), format_version=version)
        tmp.replace(src)
        file_size_after = src.stat().st_size
    return {"tensors_total": len(header["tensors"]), "tensors_migrated": migrated,
            "bytes_before": bytes_before, "bytes_after": bytes_after,
            "savings_pct": (bytes_before - bytes_after) / bytes_before * 100.0 if bytes_before else 0.0,
            "file_size_before": file_size_before, "file_size_after": file_size_after,
            "format_version": version, "dry_run": dry_run, "codec_changes": changes}
