"""hip backend of per-token fp8-e4m3 quantisation: tb_fp8_act_quant in libtbhip.so."""
import torch

from tilebench_amd import runtime as rt

rt.load_library()

_last_config = None


def run(A: torch.Tensor, **kwargs):
    global _last_config
    rt.require_device(A)
    if A.dtype != torch.float16 or A.dim() != 2:
        raise TypeError("fp8_act_quant expects a 2-D fp16 tensor")
    A = A.contiguous()
    M, K = A.shape
    Aq = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=A.device)
    sa = torch.empty((M,), dtype=torch.float32, device=A.device)
    rt.call("tb_fp8_act_quant", A.data_ptr(), Aq.data_ptr(), sa.data_ptr(), M, K, rt.stream_handle(A.device))
    _last_config = {"kernel": "fp8_quant_rows", "block": 256, "items_per_thread": max(1, -(-K // 2048))}
    return (Aq, sa)


def get_last_config():
    return _last_config
