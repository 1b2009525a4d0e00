"""hip backend of the row/column-scaled fp8 GEMM: tb_fp8_scaled_gemm in libtbhip.so.

The weight operand is consumed K-contiguous (Wq.t() is a dense [N, K] buffer in
the generator's layout, the layout torch._scaled_mm takes); any other layout is
made K-contiguous first.
"""
import torch

from tilebench_amd import runtime as rt

rt.load_library()

_last_config = None


def run(Aq: torch.Tensor, Wq: torch.Tensor, sa: torch.Tensor, sw: torch.Tensor, **kwargs):
    global _last_config
    rt.require_device(Aq, Wq, sa, sw)
    if Aq.dtype != torch.float8_e4m3fn or Wq.dtype != torch.float8_e4m3fn:
        raise TypeError("fp8_scaled_gemm expects float8_e4m3fn operands")
    M, K = Aq.shape
    K2, N = Wq.shape
    if K2 != K or tuple(sa.shape) != (M,) or tuple(sw.shape) != (N,):
        raise ValueError("fp8_scaled_gemm: operand / scale shapes do not match")
    Aq = Aq.contiguous()
    WqT = Wq.t().contiguous()
    sa = sa.to(torch.float32).contiguous()
    sw = sw.to(torch.float32).contiguous()
    Y = torch.empty((M, N), dtype=torch.bfloat16, device=Aq.device)
    rt.call("tb_fp8_scaled_gemm", Aq.data_ptr(), WqT.data_ptr(), sa.data_ptr(), sw.data_ptr(), Y.data_ptr(), M, N, K,
            rt.stream_handle(Aq.device))
    _last_config = {"kernel": "fp8_gemm_kernel", "BM": 256, "BN": 256, "BK": 128, "waves": 4}
    return Y


def get_last_config():
    return _last_config
