"""hip backend of the W4A16 GEMM: libtbhip.so's tb_w4a16_gemm family.

M <= 16 (decode): when the shape allows it, the slab decode kernel
(tb_w4a16_gemm_slabs) over a slab-contiguous copy of the packed weights,
built by tb_w4a16_repack_slabs on the first call with a weight tensor and kept
with it (keyed by its storage, dropped when the tensor is freed) -- the way the
reference's fp8 matmul keeps a column-major copy of its second operand per
operand (tilebench/benchmarks/operators/matmul_fp32_fp16_fp8/impl_torch.py:
7-18).  The weights are treated as constant while the copy lives, as there.  A
call under graph capture never builds a copy (no allocation or extra kernel
goes into the graph): without one it runs the split-K decode on the original
layout, as do shapes the slab kernel does not take.  Larger M runs the MFMA
prefill kernel.
"""
import ctypes
import weakref

import torch

from tilebench_amd import runtime as rt

rt.load_library()

_last_config = None
#: (data_ptr, K, N, device index) -> (weakref to the packed weights, slab copy)
_slab_cache: dict = {}


def slab_shape_ok(M: int, N: int, K: int, group: int) -> bool:
    """Whether the slab decode takes this shape (tb_w4a16_gemm_slabs' limits,
    within the operator's own group % 64 == 0)."""
    return 1 <= M <= 16 and N % 64 == 0 and group in (64, 128) and K in (1024, 2048, 4096) and K % (16 * group) == 0


def slab_copy(packed: torch.Tensor, K: int, N: int):
    """The slab-contiguous copy of `packed` (built on first use; None under
    graph capture when it does not exist yet)."""
    key = (packed.data_ptr(), K, N, packed.device.index)
    hit = _slab_cache.get(key)
    if hit is not None:
        ref, copy = hit
        if ref() is packed:
            return copy
        del _slab_cache[key]          # another tensor now lives at this address
    if torch.cuda.is_current_stream_capturing():
        return None
    copy = torch.empty(K * N // 2, dtype=torch.uint8, device=packed.device)
    rt.call("tb_w4a16_repack_slabs", packed.data_ptr(), copy.data_ptr(), K, N, rt.stream_handle(packed.device))
    _slab_cache[key] = (weakref.ref(packed, lambda _r, k=key: _slab_cache.pop(k, None)), copy)
    return copy


def run(A: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, group: int, *,
        slabs: bool = True, **kwargs):
    """Y = A @ dequant(packed).  `slabs=False` keeps M <= 16 on the split-K
    decode over the original layout (no per-weight copy)."""
    global _last_config
    rt.require_device()
    if A.dtype != torch.float16 or packed.dtype != torch.uint8 or zeros.dtype != torch.uint8 \
            or scales.dtype != torch.float16:
        raise TypeError("w4a16_gemm expects fp16 A/scales and uint8 packed weights/zeros")
    M, K = A.shape
    N = packed.shape[1] * 2
    if tuple(packed.shape) != (K, N // 2) or tuple(scales.shape) != (K // group, N) \
            or tuple(zeros.shape) != (K // group, N // 2):
        raise ValueError("w4a16_gemm: weight / scale / zero shapes do not match A")
    A, scales, zeros = A.contiguous(), scales.contiguous(), zeros.contiguous()
    if not packed.is_contiguous():
        packed = packed.contiguous()
    Y = torch.empty((M, N), dtype=torch.float16, device=A.device)
    stream = rt.stream_handle(A.device)
    wr = slab_copy(packed, K, N) if slabs and slab_shape_ok(M, N, K, group) else None
    if wr is not None:
        rt.call("tb_w4a16_gemm_slabs", A.data_ptr(), wr.data_ptr(), scales.data_ptr(), zeros.data_ptr(),
                Y.data_ptr(), M, N, K, group, stream)
        _last_config = {"kernel": "w4a16_slab_decode", "cols_per_block": 64, "waves": 16}
        return Y
    need = ctypes.c_int64(0)
    rt.call("tb_w4a16_workspace_size", M, N, K, group, ctypes.byref(need))
    ws = rt.workspace(need.value, A.device, stream)
    rt.call("tb_w4a16_gemm", A.data_ptr(), packed.data_ptr(), scales.data_ptr(), zeros.data_ptr(), Y.data_ptr(),
            M, N, K, group, rt.ptr(ws), need.value, stream)
    _last_config = ({"kernel": "w4a16_decode", "cols_per_block": 256, "workspace_bytes": need.value}
                    if M <= 16 else {"kernel": "w4a16_prefill", "BM": 256, "BN": 256, "BK": 64, "waves": 8})
    return Y


def get_last_config():
    return _last_config
