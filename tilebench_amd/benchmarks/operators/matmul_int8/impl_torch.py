"""PyTorch statement of matmul_int8 (reference matmul_int8/impl_torch.py:4-19).

b holds four 2-bit fields per byte; field i of packed row kb is row
i * K/4 + kb of the int8 operand, with value field - 1.  The product is taken
in fp32 as the reference does; every partial sum is an integer below 2^24 in
magnitude, so it is exact, and the result is returned as int32.
"""
import torch


def run(a: torch.Tensor, b: torch.Tensor, **kwargs):
    M, K = a.shape
    K_b, N = b.shape
    if K != 4 * K_b:
        raise ValueError("A's K dim must be 4x B's K_b dim")
    fields = [((b.to(torch.int32) >> (2 * i)) & 3) - 1 for i in range(4)]
    B = torch.cat(fields, dim=0).to(torch.float32)
    return (a.to(torch.float32) @ B).to(torch.int32)
