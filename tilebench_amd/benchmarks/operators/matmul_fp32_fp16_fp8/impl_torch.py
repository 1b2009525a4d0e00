"""PyTorch statement of matmul_fp32_fp16_fp8 (reference
matmul_fp32_fp16_fp8/impl_torch.py:10-27): a plain matmul for fp32 and fp16;
for fp8-e4m3 the product of the unit-scaled operands accumulated in fp32,
rounded to bf16 and cast back to e4m3 (what its _scaled_mm(..., out_dtype=
torch.bfloat16).to(a.dtype) computes).
"""
import torch


def run(a: torch.Tensor, b: torch.Tensor, **kwargs):
    if a.dtype == torch.float8_e4m3fn:
        return (a.to(torch.float32) @ b.to(torch.float32)).to(torch.bfloat16).to(a.dtype)
    return torch.matmul(a, b)
