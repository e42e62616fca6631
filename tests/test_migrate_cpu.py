"""migrate's rules that need no GPU (bigsmall/migrate.py:41-43, 94-108, 133-141):
a delta container is skipped; entries in kept codecs and entries whose codec
this engine does not decode (the constriction formats) stay byte for byte."""
from __future__ import annotations

import hashlib

from bigsmall_amd import container, formats
from bigsmall_amd.migrate import migrate


def _write(path, tensors, blobs, **extra_header):
    data, entries, off = b"", [], 0
    for t, b in zip(tensors, blobs):
        entries.append({**t, "compressed_bytes": len(b), "offset": off})
        data += b
        off += len(b)
    header = {"format": "bf16", "mode": "balanced", "tensor_count": len(entries), "tensors": entries,
              "codec_stats": {}, **extra_header}
    container.write_container(path, header, data, format_version=formats.BS_FORMAT_VERSION_V1)


def test_delta_container_is_not_migrated(tmp_path):
    p = tmp_path / "d.bs"
    _write(p, [{"name": "w", "shape": [4], "dtype": "bfloat16", "codec": "zstd_xor_delta", "md5": "", "extra": None}],
           [b"\x28\xb5\x2f\xfd" + bytes(12)], model_type="delta")
    digest = hashlib.sha256(p.read_bytes()).hexdigest()
    r = migrate(p)
    assert r["skipped_reason"] == "delta_container_not_migrated" and r["tensors_migrated"] == 0
    assert r["savings_pct"] == 0.0 and r["file_size_after"] == r["file_size_before"] == p.stat().st_size
    assert hashlib.sha256(p.read_bytes()).hexdigest() == digest


def test_kept_and_undecodable_entries_stay_as_they_are(tmp_path):
    p = tmp_path / "k.bs"
    ts = [{"name": "a", "shape": [3], "dtype": "bfloat16", "codec": "raw", "md5": "", "extra": None},
          {"name": "b", "shape": [3], "dtype": "bfloat16", "codec": "tied_ref", "md5": "", "extra": {"ref": "a"}},
          {"name": "c", "shape": [64], "dtype": "bfloat16", "codec": "bf16_se_rans", "md5": "", "extra": {}}]
    blobs = [b"\x01\x02\x03\x04\x05\x06", b"", bytes(range(40))]
    _write(p, ts, blobs)
    r = migrate(p, backup=False)
    assert r["tensors_migrated"] == 0 and r["codec_changes"] == {}
    assert r["bytes_after"] == r["bytes_before"] == sum(map(len, blobs))
    assert r["format_version"] == formats.BS_FORMAT_VERSION_V1
    header, off = container.read_header(p)
    data = p.read_bytes()[off:]
    for t, t0, b in zip(header["tensors"], ts, blobs):
        assert t["codec"] == t0["codec"] and data[t["offset"]:t["offset"] + t["compressed_bytes"]] == b
    assert header["codec_stats"] == {"raw": 1, "tied_ref": 1, "bf16_se_rans": 1}
