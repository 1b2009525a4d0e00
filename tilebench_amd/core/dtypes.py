"""dtype names used in configs (tilebench/core/dtypes.py:16-47)."""
from __future__ import annotations

import torch

_DTYPE_SIZE_MAP: dict[str, int] = {
    "float32": 4, "fp32": 4,
    "float16": 2, "fp16": 2,
    "bfloat16": 2, "bf16": 2,
    "int8": 1, "int16": 2, "int32": 4, "int64": 8,
    "fp8": 1, "fp8_e5m2": 1, "fp8_e4m3fn": 1,
    "float8_e5m2": 1, "float8_e4m3fn": 1,
    "int4": 1, "uint8": 1,
}

_ALIASES = {
    "float32": "float32", "fp32": "float32",
    "float16": "float16", "fp16": "float16",
    "bfloat16": "bfloat16", "bf16": "bfloat16",
    "int8": "int8", "int16": "int16", "int32": "int32", "int64": "int64", "uint8": "uint8",
    "fp8": "float8_e5m2", "fp8_e5m2": "float8_e5m2", "fp8_e4m3fn": "float8_e4m3fn",
}


def dtype_size(dtype_name: str) -> int:
    return _DTYPE_SIZE_MAP.get(dtype_name.lower(), 4)


def resolve_dtype(dtype_name: str) -> torch.dtype:
    key = dtype_name.lower()
    candidate = _ALIASES.get(key, key)
    if hasattr(torch, candidate):
        return getattr(torch, candidate)
    raise ValueError(f"Unsupported dtype '{dtype_name}' for this environment.")
