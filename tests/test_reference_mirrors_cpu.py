"""Mirrors of the reference's own tests of the container, version-error and
tiny-tensor behaviour that the drop-in keeps, and of the streaming model's helpers (no GPU needed):
  tests/test_version_errors.py:12-72, tests/test_format_v2.py:55-103,
  tests/test_raw_tiny.py:30-110, tests/test_streaming_inference.py:14-55.
The decode half of the tiny-tensor round trip runs on the GPU in the reference's
API tests; here the raw blobs are compared byte for byte."""
from __future__ import annotations

import struct

import pytest
import torch


def _write_future(path):
    from bigsmall_amd import container
    header_bytes = b"{}"
    with open(path, "wb") as f:
        f.write(container.MAGIC)
        f.write(struct.pack("<H", 99))
        f.write(struct.pack("<I", len(header_bytes)))
        f.write(header_bytes)


def test_version_error_importable_from_package():
    import bigsmall_amd
    assert issubclass(bigsmall_amd.BigSmallVersionError, Exception)


def test_unsupported_container_version_raises_versionerror(tmp_path):
    from bigsmall_amd import BigSmallVersionError, container
    p = tmp_path / "future.bs"
    _write_future(p)
    with pytest.raises(BigSmallVersionError) as excinfo:
        container.read_header(p)
    msg = str(excinfo.value)
    assert "pip install --upgrade bigsmall" in msg
    assert "requires bigsmall >= 2.4.0" in msg


def test_unknown_codec_in_decoder_raises_versionerror():
    from bigsmall_amd import BigSmallVersionError
    from bigsmall_amd.decoder import _decode_blob
    meta = {"name": "x", "shape": [4], "dtype": "BF16", "codec": "future_codec_v9", "special": None,
            "compressed_bytes": 8, "offset": 0, "md5": "0" * 32, "extra": None}
    with pytest.raises(BigSmallVersionError) as excinfo:
        _decode_blob(meta, b"\x00" * 8)
    assert "pip install --upgrade bigsmall" in str(excinfo.value)
    assert "future_codec_v9" in str(excinfo.value)


def test_versionerror_message_format():
    from bigsmall_amd import BigSmallVersionError
    msg = str(BigSmallVersionError(required="3.0.0", installed="2.4.0", detail="hypothetical"))
    for part in ("requires bigsmall >= 3.0.0", "you have 2.4.0", "pip install --upgrade bigsmall", "hypothetical"):
        assert part in msg


def test_v2_writer_emits_v2_and_reads_back(tmp_path):
    from bigsmall_amd import container
    from bigsmall_amd.formats import BS_FORMAT_VERSION_V2
    p = tmp_path / "synthetic.bs"
    header = {"format": "bf16", "mode": "balanced", "model_type": "llm", "base_model": None, "tensor_count": 0,
              "tensors": [], "safetensors_metadata": None}
    container.write_container(p, header, data=b"", format_version=BS_FORMAT_VERSION_V2)
    with open(p, "rb") as f:
        f.seek(4)
        assert struct.unpack("<H", f.read(2))[0] == BS_FORMAT_VERSION_V2
    h, _ = container.read_header(p)
    assert h["_format_version"] == BS_FORMAT_VERSION_V2


def test_unsupported_version_rejected_clearly(tmp_path):
    from bigsmall_amd import BigSmallVersionError, container
    p = tmp_path / "future.bs"
    _write_future(p)
    with pytest.raises(BigSmallVersionError, match="pip install --upgrade bigsmall"):
        container.read_header(p)


def _tiny_model():
    torch.manual_seed(0)
    return {"tiny.bias": torch.randn(128, dtype=torch.bfloat16),
            "very_tiny.scale": torch.tensor([1.5, -0.25], dtype=torch.float32),
            "norm.weight": torch.randn(2048, dtype=torch.bfloat16),
            "matrix.weight": torch.randn(512, 512, dtype=torch.bfloat16)}


def test_tiny_tensor_uses_raw_codec(tmp_path):
    from safetensors.torch import save_file

    import bigsmall_amd
    from bigsmall_amd import container
    src = tmp_path / "model.safetensors"
    tensors = _tiny_model()
    save_file(tensors, str(src))
    bs = tmp_path / "model.bs"
    bigsmall_amd.compress(src, bs)
    header, off = container.read_header(bs)
    by = {t["name"]: t for t in header["tensors"]}
    assert by["tiny.bias"]["codec"] == "raw" and by["very_tiny.scale"]["codec"] == "raw"
    assert by["tiny.bias"]["compressed_bytes"] == 256 and by["very_tiny.scale"]["compressed_bytes"] == 8
    assert by["norm.weight"]["codec"] != "raw" and by["matrix.weight"]["codec"] != "raw"
    for i, t in enumerate(header["tensors"]):
        if t["codec"] == "raw":
            want = tensors[t["name"]].contiguous().view(torch.uint8).numpy().tobytes()
            assert container.read_blob(bs, header, off, i) == want


def test_threshold_boundary(tmp_path):
    from safetensors.torch import save_file

    import bigsmall_amd
    from bigsmall_amd import container, encoder
    threshold = encoder.RAW_TINY_THRESHOLD
    src = tmp_path / "model.safetensors"
    save_file({"at_threshold.weight": torch.zeros(threshold // 2, dtype=torch.bfloat16),
               "below_threshold.weight": torch.zeros(threshold // 2 - 1, dtype=torch.bfloat16)}, str(src))
    bs = tmp_path / "model.bs"
    bigsmall_amd.compress(src, bs)
    header, _ = container.read_header(bs)
    codec = {t["name"]: t["codec"] for t in header["tensors"]}
    assert codec["below_threshold.weight"] == "raw"
    assert codec["at_threshold.weight"] != "raw"


# tests/test_streaming_inference.py:14-55: the streaming model's helpers
def test_streaming_inference_imports():
    import bigsmall_amd.streaming_inference  # noqa: F401


def test_set_param_data_swaps_parameter():
    from torch import nn

    from bigsmall_amd.streaming_inference import _set_param_data
    m = nn.Linear(4, 4)
    _set_param_data(m, "weight", torch.zeros(4, 4))
    assert torch.equal(m.weight, torch.zeros(4, 4)) and isinstance(m.weight, nn.Parameter)


def test_set_param_data_nested_index():
    from torch import nn

    from bigsmall_amd.streaming_inference import _set_param_data
    m = nn.ModuleList([nn.Linear(2, 2), nn.Linear(2, 2)])
    _set_param_data(m, "1.weight", torch.eye(2))
    assert torch.equal(m[1].weight, torch.eye(2))


def test_layer_prefix_format():
    from bigsmall_amd.streaming_inference import _layer_prefix
    assert _layer_prefix(0) == "model.layers.0."
    assert _layer_prefix(31) == "model.layers.31."
    assert _layer_prefix(5, "h.{}") == "h.5."
