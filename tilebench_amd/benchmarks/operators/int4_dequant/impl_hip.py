"""hip backend of int4 group-wise dequantisation: tb_int4_dequant in libtbhip.so.

Same run() signature as impl_torch.run (the reference engine calls
impl.run(*inputs), tilebench/core/engine.py:347-348).
"""
import torch

from tilebench_amd import runtime as rt

rt.load_library()

_last_config = None


def run(packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, K: int, N: int, group: int, **kwargs):
    global _last_config
    rt.require_device(packed, scales, zeros)
    if packed.dtype != torch.uint8 or zeros.dtype != torch.uint8 or scales.dtype != torch.float16:
        raise TypeError("int4_dequant expects uint8 packed/zeros and fp16 scales")
    if tuple(packed.shape) != (K, N // 2) or tuple(scales.shape) != (K // group, N) \
            or tuple(zeros.shape) != (K // group, N // 2):
        raise ValueError(f"int4_dequant: shapes {tuple(packed.shape)}, {tuple(scales.shape)}, "
                         f"{tuple(zeros.shape)} do not match K={K} N={N} group={group}")
    packed, scales, zeros = packed.contiguous(), scales.contiguous(), zeros.contiguous()
    out = torch.empty((K, N), dtype=torch.float16, device=packed.device)
    rt.call("tb_int4_dequant", packed.data_ptr(), scales.data_ptr(), zeros.data_ptr(), out.data_ptr(),
            K, N, group, rt.stream_handle(packed.device))
    _last_config = {"kernel": "int4_dequant_vec" if N % 8 == 0 and group % 8 == 0 else "int4_dequant_scalar",
                    "rows_per_thread": 8, "cols_per_thread": 8}
    return out


def get_last_config():
    return _last_config
