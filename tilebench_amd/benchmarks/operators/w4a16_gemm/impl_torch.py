"""PyTorch reference of the W4A16 GEMM.

The reference's fp16 GEMM (matmul_fp32_fp16_fp8/impl_torch.py:21-27, torch.matmul)
applied to the int4 weights dequantised exactly as in int4_dequant/impl_torch.py:
Y = fp16(A.float() @ dequant(W).float()), fp32 accumulation.  Weights in the
decode's slab layout ([N/64, K/32, 1024], tilebench_amd.formats) are first
mapped back to the packed [K, N/2] layout.
"""
import torch

from tilebench_amd.benchmarks.operators.int4_dequant.impl_torch import dequant
from tilebench_amd.formats import w4a16_from_slabs


def run(A: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, group: int, **kwargs):
    if packed.dim() == 3:
        packed = w4a16_from_slabs(packed)
    W = dequant(packed, scales, zeros, group)
    return (A.to(torch.float32) @ W.to(torch.float32)).to(torch.float16)
