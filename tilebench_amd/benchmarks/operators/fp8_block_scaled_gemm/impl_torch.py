"""PyTorch reference of the block-scaled fp8 GEMM.

Both operands are dequantised with the reference's block-scale map
(weight_dequant/impl_torch.py:4-8: X * S[i//T, j//T], T = 128) -- the weights
WqT [N, K] by sw [N/128, K/128], the activations Aq [M, K] by sa [K/128, M]
(one scale per token and 128 channels) -- and multiplied in fp32 as the
reference's fp8 GEMM accumulates (matmul_fp32_fp16_fp8/impl_torch.py:10-26),
then rounded once to bf16.  Each product Aq * Wq is exact in fp32, so this
differs from the blockwise sum only by fp32 accumulation order.
"""
import torch

BLOCK = 128


def run(Aq: torch.Tensor, WqT: torch.Tensor, sa: torch.Tensor, sw: torch.Tensor, **kwargs):
    M, K = Aq.shape
    N = WqT.shape[0]
    a = Aq.to(torch.float32) * sa.t().repeat_interleave(BLOCK, dim=1)
    s_w = sw.repeat_interleave(BLOCK, dim=0)[:N].repeat_interleave(BLOCK, dim=1)
    w = WqT.to(torch.float32) * s_w
    return (a @ w.t()).to(torch.bfloat16)
