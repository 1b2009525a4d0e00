"""PyTorch reference of dequantize_rowwise (tilebench/benchmarks/operators/dequantize_rowwise/impl_torch.py:4-7):
y = fp16((state_x[r] * x[r, c]) * (1/127)), evaluated left to right in fp32."""
import torch


def run(x: torch.Tensor, state_x: torch.Tensor, **kwargs):
    prod = state_x[:, None] * x           # int8 promotes to fp32
    return (prod * (1.0 / 127.0)).to(torch.float16)
