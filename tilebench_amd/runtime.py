"""ctypes binding of libtbhip.so, the C ABI declared in include/tbhip.h.

The library is built in-tree (``python -m tilebench_amd.build``) and loaded on
first use.  Nothing here falls back to another implementation: a missing
library, a missing symbol or a host without a gfx950 device raises, so a caller
never silently measures or verifies something else.

Every entry point is called with raw ``data_ptr()`` values and the HIP stream
of the current torch stream; a non-zero status raises ``RuntimeError`` carrying
the library's own message (``tb_last_error``), or ``ValueError`` for shape and
alignment errors (the reference engine treats both as a failed backend,
tilebench/core/engine.py:361-366).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libtbhip.so"

TB_OK = 0
TB_E_INVALID = 1
TB_E_ALIGN = 2
TB_E_HIP = 3
TB_E_WORKSPACE = 4

_c_i64 = ctypes.c_int64
_c_p = ctypes.c_void_p
_c_int = ctypes.c_int
_c_u32 = ctypes.c_uint32

#: symbol -> argtypes (every entry point returns an int status).
SIGNATURES: dict[str, list] = {
    "tb_int4_dequant": [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p],
    "tb_moe_topk_gating": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_p],
    "tb_fp8_act_quant": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_p],
    "tb_w4a16_gemm": [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p],
    "tb_w4a16_workspace_size": [_c_i64, _c_i64, _c_i64, _c_i64, ctypes.POINTER(_c_i64)],
    "tb_w4a16_gemm_noalloc": [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p],
    "tb_w4a16_repack_slabs": [_c_p, _c_p, _c_i64, _c_i64, _c_p],
    "tb_w4a16_gemm_slabs": [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p],
    "tb_moe_w4a16_grouped_gemm": [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p],
    "tb_moe_align": [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p],
    "tb_moe_w4a16_gate_up": [_c_p] * 7 + [_c_i64] * 6 + [_c_p],
    "tb_moe_w4a16_down": [_c_p] * 8 + [_c_i64] * 5 + [_c_p],
    "tb_moe_combine": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p],
    "tb_fused_moe_w4a16_workspace_size": [_c_i64] * 5 + [ctypes.POINTER(_c_i64)],
    "tb_fused_moe_w4a16": [_c_p] * 9 + [_c_i64] * 7 + [_c_p, _c_i64, _c_p],
    "tb_fp8_scaled_gemm": [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p],
    "tb_fp8_act_quant_blocks": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_p],
    "tb_fp8_block_gemm": [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p],
    "tb_weight_dequant": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_p],
    "tb_dequantize_rowwise": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_p],
    "tb_quantize_global": [_c_p, _c_p, _c_i64, _c_p],
    "tb_matmul_int8": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p],
    "tb_matmul": [_c_int, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p],
    "tb_matmul_fp8_bt": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p],
    "tb_matmul_workspace_size": [_c_int, _c_i64, _c_i64, _c_i64, ctypes.POINTER(_c_i64)],
    "tb_l2_flush": [_c_p, _c_i64, _c_u32, _c_p],
    "tb_probe_copy": [_c_p, _c_p, _c_i64, _c_p],
    "tb_probe_read": [_c_p, _c_i64, _c_u32, _c_p, _c_p],
    "tb_probe_mfma": [_c_int, _c_i64, _c_i64, _c_p, _c_p],
    "tb_probe_clock": [_c_i64, _c_i64, _c_p, _c_p, _c_p],
}

#: symbols returning a C string
STRING_SYMBOLS = ("tb_version", "tb_last_error")

_lib = None


class HipBackendUnavailable(ImportError):
    """libtbhip.so is missing or cannot run here (no gfx950 device)."""


def load_library(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load libtbhip.so and declare its signatures (no GPU needed)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise HipBackendUnavailable(
            f"{p} is not built; run `python -m tilebench_amd.build` (or __graft_entry__.build())")
    lib = ctypes.CDLL(str(p))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    for name in STRING_SYMBOLS:
        fn = getattr(lib, name)
        fn.argtypes = []
        fn.restype = ctypes.c_char_p
    if path is None:
        _lib = lib
    return lib


def version() -> str:
    return load_library().tb_version().decode()


def check(status: int, what: str) -> None:
    """Raise on a non-zero status with the library's message."""
    if status == TB_OK:
        return
    msg = load_library().tb_last_error().decode(errors="replace")
    if status in (TB_E_INVALID, TB_E_ALIGN, TB_E_WORKSPACE):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (status {status})")


_device_checked = False


def require_device(*tensors) -> None:
    """Fail loudly unless the current device is a gfx950 GPU and every given
    tensor lives on it.  The kernels take raw addresses and launch on the
    current device: a host tensor's pointer would reach a kernel as a device
    address, so it is refused here with a ValueError instead."""
    global _device_checked
    import torch

    if not _device_checked:
        if not torch.cuda.is_available() or not torch.version.hip:
            raise HipBackendUnavailable("the hip backend needs a ROCm GPU (torch.cuda is unavailable)")
        arch = (getattr(torch.cuda.get_device_properties(torch.cuda.current_device()), "gcnArchName", "") or "")
        if not arch.startswith("gfx950"):
            raise HipBackendUnavailable(f"libtbhip.so is built for gfx950, the device is {arch!r}")
        _device_checked = True
    if tensors:
        here = torch.cuda.current_device()
        for i, t in enumerate(tensors):
            if isinstance(t, torch.Tensor) and (t.device.type != "cuda" or t.device.index != here):
                raise ValueError(f"hip backend: input {i} is on {t.device}, the kernels run on cuda:{here}")


def stream_handle(device=None) -> int:
    """Raw hipStream_t of torch's current stream."""
    import torch

    return torch.cuda.current_stream(device).cuda_stream


def call(name: str, *args) -> None:
    """Call an entry point with (already converted) arguments and check it."""
    lib = load_library()
    check(getattr(lib, name)(*args), name)


def ptr(t) -> int:
    """data_ptr of a tensor (0 for None)."""
    return 0 if t is None else t.data_ptr()


_workspaces: dict = {}
#: every workspace ever handed out, kept alive until the process ends
_retired: list = []


def matmul_workspace_size(dtype: int, M: int, N: int, K: int) -> int:
    """Bytes of workspace tb_matmul (dtype 0 fp32, 1 fp16, 2 fp8) or
    tb_matmul_int8 (dtype 3) needs for this shape."""
    out = ctypes.c_int64(0)
    call("tb_matmul_workspace_size", dtype, M, N, K, ctypes.byref(out))
    return int(out.value)


def workspace(nbytes: int, device, stream: int):
    """A zero-filled device workspace of at least `nbytes`, cached per device.

    Kernels that use one restore every counter they touch to zero, so the
    buffer is zero-filled only when it is first allocated (outside any graph
    capture: the engine and the bench always run a call eagerly first).  One
    buffer per device serves calls issued in order on one stream (graph
    replays included); calls running concurrently on several streams of one
    device would race on it and are not supported.

    When a call needs more than the cached buffer holds, a larger one becomes
    the cached buffer and the old one is kept alive (never returned to the
    caching allocator): a graph captured earlier holds the old buffer's raw
    address, and its replays must keep finding a live, zeroed workspace there."""
    import torch

    del stream  # calls are serialised on one stream; see the docstring
    if nbytes <= 0:
        return None
    key = str(device)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("workspace must be allocated before graph capture (run the op once eagerly)")
        new = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        if buf is not None:
            _retired.append(buf)
        _workspaces[key] = buf = new
    return buf
