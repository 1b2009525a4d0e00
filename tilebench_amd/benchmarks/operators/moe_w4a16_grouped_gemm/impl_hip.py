"""hip backend of the grouped MoE W4A16 GEMM: tb_moe_w4a16_grouped_gemm in libtbhip.so."""
import torch

from tilebench_amd import runtime as rt

rt.load_library()

_last_config = None


def run(A: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, offsets: torch.Tensor,
        group: int, **kwargs):
    global _last_config
    rt.require_device(A, packed, scales, zeros, offsets)
    if A.dtype != torch.float16 or packed.dtype != torch.uint8 or zeros.dtype != torch.uint8 \
            or scales.dtype != torch.float16:
        raise TypeError("moe_w4a16_grouped_gemm expects fp16 A/scales and uint8 packed weights/zeros")
    R, K = A.shape
    E, K2, half_n = packed.shape
    N = half_n * 2
    if K2 != K or tuple(scales.shape) != (E, K // group, N) or tuple(zeros.shape) != (E, K // group, N // 2) \
            or tuple(offsets.shape) != (E + 1,):
        raise ValueError("moe_w4a16_grouped_gemm: expert weight / scale / zero / offset shapes do not match A")
    A, packed, scales, zeros = A.contiguous(), packed.contiguous(), scales.contiguous(), zeros.contiguous()
    offsets = offsets.to(device=A.device, dtype=torch.int32).contiguous()
    # offsets run from 0 to R, so every row of Y belongs to one segment and is written
    Y = torch.empty((R, N), dtype=torch.float16, device=A.device)
    rt.call("tb_moe_w4a16_grouped_gemm", A.data_ptr(), packed.data_ptr(), scales.data_ptr(), zeros.data_ptr(),
            offsets.data_ptr(), Y.data_ptr(), R, E, N, K, group, rt.stream_handle(A.device))
    _last_config = {"kernel": "w4a16_grouped", "BM": 256, "BN": 256, "BK": 64, "waves": 4,
                    "last_tiles": "256 x 128 for <= 128 columns"}
    return Y


def get_last_config():
    return _last_config
