"""hip backend of the W4A16 GEMM: tb_w4a16_gemm in libtbhip.so.

M <= 16 runs the split-K decode kernel (with a cached, self-cleaning
workspace), larger M the MFMA prefill kernel.
"""
import ctypes

import torch

from tilebench_amd import runtime as rt

rt.load_library()

_last_config = None


def run(A: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, group: int, **kwargs):
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
    A, packed, scales, zeros = A.contiguous(), packed.contiguous(), scales.contiguous(), zeros.contiguous()
    Y = torch.empty((M, N), dtype=torch.float16, device=A.device)
    need = ctypes.c_int64(0)
    rt.call("tb_w4a16_workspace_size", M, N, K, group, ctypes.byref(need))
    stream = rt.stream_handle(A.device)
    ws = rt.workspace(need.value, A.device, stream)
    rt.call("tb_w4a16_gemm", A.data_ptr(), packed.data_ptr(), scales.data_ptr(), zeros.data_ptr(), Y.data_ptr(),
            M, N, K, group, rt.ptr(ws), need.value, stream)
    _last_config = ({"kernel": "w4a16_decode", "cols_per_block": 256, "workspace_bytes": need.value}
                    if M <= 16 else {"kernel": "w4a16_prefill", "BM": 256, "BN": 256, "BK": 64, "waves": 8})
    return Y


def get_last_config():
    return _last_config
