"""PyTorch reference of the row/column-scaled fp8 GEMM.

The reference's fp8 path (matmul_fp32_fp16_fp8/impl_torch.py:10-26) is
torch._scaled_mm(a, b_colmajor, scale_a, scale_b, out_dtype=bf16) with unit
scales.  Here the scales are a per-row sa [M] and a per-column sw [N]; since
torch's CPU _scaled_mm only takes per-tensor scales, the product is formed as
the fp32 GEMM of the decoded e4m3 operands (every product exact in fp32) scaled
by sa[m] * sw[n] and rounded once to bf16.
"""
import torch


def run(Aq: torch.Tensor, Wq: torch.Tensor, sa: torch.Tensor, sw: torch.Tensor, **kwargs):
    acc = Aq.to(torch.float32) @ Wq.to(torch.float32)
    return (acc * sa[:, None] * sw[None, :]).to(torch.bfloat16)
