"""PyTorch reference of int4 group-wise dequantisation.

Follows the reference's dequantisation operator (weight_dequant/impl_torch.py:4-8:
an elementwise product with a scale picked by index arithmetic) for int4 codes
with zero-points: out[k, n] = fp16((q[k,n] - z[k//G, n]) * s[k//G, n]).  Codes are
unpacked low nibble first, like the sub-byte unpack of matmul_int8/impl_torch.py:10-14.
Works on any device.
"""
import torch


def unpack_int4(p: torch.Tensor) -> torch.Tensor:
    """uint8 [..., C/2] -> int16 codes [..., C]: byte j holds codes 2j (bits 0-3) and 2j+1 (bits 4-7)."""
    p = p.to(torch.int16)
    return torch.stack((p & 0xF, p >> 4), dim=-1).reshape(*p.shape[:-1], -1)


def dequant(packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, group: int) -> torch.Tensor:
    q = unpack_int4(packed)
    z = unpack_int4(zeros).repeat_interleave(group, dim=-2)
    s = scales.repeat_interleave(group, dim=-2)
    # (q - z) is exact in fp16; fp16 * fp16 rounds the exact product once.
    return (q - z).to(torch.float16) * s


def run(packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, K: int, N: int, group: int, **kwargs):
    return dequant(packed, scales, zeros, group)
