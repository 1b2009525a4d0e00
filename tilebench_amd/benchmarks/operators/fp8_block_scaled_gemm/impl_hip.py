"""hip backend of the block-scaled fp8 GEMM: tb_fp8_block_gemm in libtbhip.so.

Operands as a block-scaled checkpoint and the per-block activation quantiser
give them: Aq e4m3 [M, K], WqT e4m3 [N, K] (the checkpoint's `weight`), sa fp32
[K/128, M] (tb_fp8_act_quant_blocks), sw fp32 [ceil(N/128), K/128] (the
checkpoint's `weight_scale_inv`).
"""
import torch

from tilebench_amd import runtime as rt

rt.load_library()

_last_config = None


def run(Aq: torch.Tensor, WqT: torch.Tensor, sa: torch.Tensor, sw: torch.Tensor, **kwargs):
    global _last_config
    rt.require_device(Aq, WqT, sa, sw)
    if Aq.dtype != torch.float8_e4m3fn or WqT.dtype != torch.float8_e4m3fn:
        raise TypeError("fp8_block_scaled_gemm expects float8_e4m3fn operands")
    M, K = Aq.shape
    N, K2 = WqT.shape
    if K2 != K or K % 128 or tuple(sa.shape) != (K // 128, M) or tuple(sw.shape) != (-(-N // 128), K // 128):
        raise ValueError("fp8_block_scaled_gemm: operand / scale shapes do not match (need K % 128 == 0, "
                         "sa [K/128, M], sw [ceil(N/128), K/128])")
    Aq, WqT = Aq.contiguous(), WqT.contiguous()
    sa = sa.to(torch.float32).contiguous()
    sw = sw.to(torch.float32).contiguous()
    Y = torch.empty((M, N), dtype=torch.bfloat16, device=Aq.device)
    rt.call("tb_fp8_block_gemm", Aq.data_ptr(), WqT.data_ptr(), sa.data_ptr(), sw.data_ptr(), Y.data_ptr(), M, N, K,
            rt.stream_handle(Aq.device))
    _last_config = {"kernel": "fp8_block_gemm", "BM": 256, "BN": 256, "BK": 128, "waves": 8}
    return Y


def get_last_config():
    return _last_config
