"""hip backend of per-token, per-128-channel fp8-e4m3 quantisation:
tb_fp8_act_quant_blocks in libtbhip.so (sa block-major, [K/128, M])."""
import torch

from tilebench_amd import runtime as rt

rt.load_library()

_last_config = None


def run(A: torch.Tensor, **kwargs):
    global _last_config
    rt.require_device(A)
    if A.dtype != torch.float16 or A.dim() != 2:
        raise TypeError("fp8_act_quant_blocks expects a 2-D fp16 tensor")
    M, K = A.shape
    if K % 128:
        raise ValueError(f"fp8_act_quant_blocks: K = {K} is not a multiple of 128")
    A = A.contiguous()
    Aq = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=A.device)
    sa = torch.empty((K // 128, M), dtype=torch.float32, device=A.device)
    rt.call("tb_fp8_act_quant_blocks", A.data_ptr(), Aq.data_ptr(), sa.data_ptr(), M, K, rt.stream_handle(A.device))
    _last_config = {"kernel": "fp8_quant_blocks", "lanes_per_block": 16, "block": 128}
    return (Aq, sa)


def get_last_config():
    return _last_config
