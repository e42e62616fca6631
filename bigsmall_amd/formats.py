"""Container format versions and dtype tables (mirrors bigsmall/formats.py:10-74)."""
from __future__ import annotations

BS_FORMAT_VERSION_V1 = 1
BS_FORMAT_VERSION_V2 = 2
BS_FORMAT_VERSION = BS_FORMAT_VERSION_V1
BS_SUPPORTED_FORMAT_VERSIONS = frozenset({BS_FORMAT_VERSION_V1, BS_FORMAT_VERSION_V2})
# codecs that need a version-2 container: the reference's (encoder.py:482-491)
# and this engine's GPU formats
V2_CODECS = frozenset({"bf16_chunked_v1", "fp8_chunked_v1", "bf16_chunked_tans_v1", "fp8_chunked_tans_v1",
                       "bf16_parallel_v1", "bf16_sparsity_v1", "fp2_residual_v1"})

SAFETENSORS_TO_FORMAT = {"F32": "fp32", "F16": "fp16", "BF16": "bf16", "F8_E4M3": "fp8", "F8_E5M2": "fp8", "F4": "fp4"}

DTYPE_BYTES = {
    "F32": 4, "float32": 4, "F16": 2, "float16": 2, "BF16": 2, "bfloat16": 2,
    "F8_E4M3": 1, "float8_e4m3fn": 1, "F8_E5M2": 1, "float8_e5m2": 1,
    "I64": 8, "int64": 8, "I32": 4, "int32": 4, "I16": 2, "int16": 2, "I8": 1, "int8": 1,
    "U8": 1, "uint8": 1, "BOOL": 1, "bool": 1,
}


def detect_format_from_dtype(dtype_str: str) -> str:
    """bigsmall/formats.py:44-64."""
    s = dtype_str
    if s in SAFETENSORS_TO_FORMAT:
        return SAFETENSORS_TO_FORMAT[s]
    s_low = s.lower().replace("torch.", "")
    if s_low in ("float32", "f32", "fp32"):
        return "fp32"
    if s_low in ("float16", "f16", "fp16", "half"):
        return "fp16"
    if s_low in ("bfloat16", "bf16"):
        return "bf16"
    if "float8" in s_low or s_low == "fp8":
        return "fp8"
    if "float4" in s_low or s_low == "fp4":
        return "fp4"
    raise ValueError(f"Unknown dtype for BigSmall: {dtype_str}")


def torch_dtype(dtype_str: str):
    import torch
    table = {
        "F32": torch.float32, "float32": torch.float32, "F16": torch.float16, "float16": torch.float16,
        "BF16": torch.bfloat16, "bfloat16": torch.bfloat16,
        "F8_E4M3": torch.float8_e4m3fn, "float8_e4m3fn": torch.float8_e4m3fn,
        "F8_E5M2": torch.float8_e5m2, "float8_e5m2": torch.float8_e5m2,
        "I64": torch.int64, "int64": torch.int64, "I32": torch.int32, "int32": torch.int32,
        "I16": torch.int16, "int16": torch.int16, "I8": torch.int8, "int8": torch.int8,
        "U8": torch.uint8, "uint8": torch.uint8, "BOOL": torch.bool, "bool": torch.bool,
    }
    return table[dtype_str]
