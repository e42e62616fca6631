"""CPU checks for the zstd-coded entries (no GPU needed).

- the oracle (libzstd through oracle.zstd_lib) against hand-built frames whose
  meaning RFC 8878 fixes: an empty raw block, an RLE block, two raw blocks, a
  skippable frame between two frames;
- the host-side framing readers of the product (Frame_Content_Size for every
  field width, the lowcard blob layout of bigsmall/codecs/special.py:58-64)
  against frames and blobs written the way the reference writes them;
- the restated lowcard encoder against its decoder and the reference's
  framing rules (sorted distinct values, uint8 indices, 256-value limit).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import zstd_lib

pytestmark = pytest.mark.skipif(not zstd_lib.available(), reason="libzstd is not installed")

KNOWN = zstd_lib.KNOWN_FRAMES


@pytest.mark.parametrize("name", sorted(KNOWN))
def test_oracle_on_hand_built_frames(name):
    frame, want = KNOWN[name]
    assert zstd_lib.decompress(frame, len(want)) == want


@pytest.mark.parametrize("n", [0, 1, 255, 256, 300, 65791, 65792, 70000, 5_000_000])
def test_frame_content_size_every_field_width(n):
    from bigsmall_amd.codecs.zstd_gpu import frame_content_size
    data = bytes(np.random.default_rng(n).integers(0, 4, n, dtype=np.uint8))
    frame = zstd_lib.compress(data, 3)
    assert frame_content_size(frame) == n
    assert zstd_lib.decompress(frame, n) == data
    assert frame_content_size(zstd_lib.compress(data, 3, content_size=False)) is None


def test_frame_content_size_known_frames():
    from bigsmall_amd.codecs.zstd_gpu import frame_content_size
    assert frame_content_size(KNOWN["rle"][0]) == 5
    assert frame_content_size(KNOWN["no_fcs"][0]) is None
    with pytest.raises(ValueError):
        frame_content_size(b"\x00" * 8)


@pytest.mark.parametrize("item_bytes", [1, 2, 4])
def test_lowcard_blob_layout(item_bytes):
    from bigsmall_amd.codecs.zstd_gpu import parse_lowcard
    rng = np.random.default_rng(item_bytes)
    dt = {1: np.uint8, 2: np.uint16, 4: np.uint32}[item_bytes]
    first = 100 if item_bytes == 1 else 0x3F70 if item_bytes == 2 else 0x3F800000
    values = rng.choice(np.arange(first, first + 16, dtype=dt), 4096, p=np.linspace(1, 3, 16) / np.linspace(1, 3, 16).sum())
    raw = values.astype(dt).tobytes()
    blob, extras = zstd_lib.encode_lowcard(raw, item_bytes)
    lc = parse_lowcard(blob)
    assert (lc.item_bytes, lc.n_unique, lc.n_elem) == (item_bytes, 16, 4096) == (extras["item_bytes"],
                                                                                extras["n_unique"], 4096)
    table = np.frombuffer(blob[lc.lut_off:lc.lut_off + 16 * item_bytes], dt)
    assert np.array_equal(table, np.unique(values))                     # sorted distinct values
    idx = np.frombuffer(zstd_lib.decompress(blob[lc.idx_off:lc.idx_off + lc.idx_len], 4096), np.uint8)
    assert np.array_equal(table[idx], values)
    assert zstd_lib.decode_lowcard(blob, len(raw)) == raw
    with pytest.raises(ValueError):
        parse_lowcard(blob[:lc.idx_off + lc.idx_len])                  # element count cut off


def test_lowcard_rejects_more_than_256_values():
    raw = np.arange(300, dtype=np.uint16).tobytes()
    with pytest.raises(ValueError):
        zstd_lib.encode_lowcard(raw, 2)
