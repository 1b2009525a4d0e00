"""dtype names used in operator configs (the names of tilebench/core/dtypes.py:
16-47, where a bare "fp8" means e5m2 and an unknown name counts 4 bytes)."""
from __future__ import annotations

import functools

import torch

#: config name -> attribute of torch naming the dtype (names not listed are looked up as given)
_TORCH_NAME = {"fp32": "float32", "fp16": "float16", "bf16": "bfloat16", "fp8": "float8_e5m2",
               "fp8_e5m2": "float8_e5m2", "fp8_e4m3fn": "float8_e4m3fn"}
#: storage bytes of names that are not torch dtypes (packed int4 is counted per storage byte)
_STORAGE_ONLY = {"int4": 1}


def resolve_dtype(dtype_name: str) -> torch.dtype:
    key = dtype_name.lower()
    dt = getattr(torch, _TORCH_NAME.get(key, key), None)
    if not isinstance(dt, torch.dtype):
        raise ValueError(f"dtype {dtype_name!r} is not a dtype of this torch build")
    return dt


@functools.lru_cache(maxsize=None)
def dtype_size(dtype_name: str) -> int:
    key = dtype_name.lower()
    if key in _STORAGE_ONLY:
        return _STORAGE_ONLY[key]
    try:
        return torch.empty((), dtype=resolve_dtype(key)).element_size()
    except ValueError:
        return 4
