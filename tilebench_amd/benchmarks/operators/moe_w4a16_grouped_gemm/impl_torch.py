"""PyTorch reference of the grouped MoE W4A16 GEMM.

Rows offsets[e]:offsets[e+1] of the expert-sorted activations use expert e's
int4 weights: Y_e = fp16(A_e.float() @ dequant(W_e).float()), i.e. the W4A16
GEMM reference (w4a16_gemm/impl_torch.py) applied per expert segment.
"""
import torch

from tilebench_amd.benchmarks.operators.int4_dequant.impl_torch import dequant


def run(A: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, offsets: torch.Tensor,
        group: int, **kwargs):
    off = offsets.to("cpu").tolist()
    Y = torch.zeros((A.shape[0], packed.shape[-1] * 2), dtype=torch.float16, device=A.device)
    for e in range(packed.shape[0]):
        lo, hi = off[e], off[e + 1]
        if hi > lo:
            W = dequant(packed[e], scales[e], zeros[e], group)
            Y[lo:hi] = (A[lo:hi].to(torch.float32) @ W.to(torch.float32)).to(torch.float16)
    return Y
