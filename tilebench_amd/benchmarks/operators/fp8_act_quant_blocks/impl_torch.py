"""PyTorch reference of per-token, per-128-channel fp8-e4m3 quantisation.

The per-token rule of fp8_act_quant/impl_torch.py applied to every block of 128
consecutive channels of a row (the reference's block map, weight_dequant/
impl_torch.py:4-8, S[i//T, j//T] with T = 128, seen from the activation side):
sa[kb, m] = fp32(max |A[m, 128 kb : 128 kb + 128]|) / 448 and
Aq = (A.float() / sa).to(float8_e4m3fn); an all-zero block has sa = 0 and 0xFF
codes.  sa is returned block-major, [K/128, M].
"""
import torch

BLOCK = 128


def run(A: torch.Tensor, **kwargs):
    M, K = A.shape
    if K % BLOCK:
        raise ValueError(f"K = {K} is not a multiple of {BLOCK}")
    blocks = A.reshape(M, K // BLOCK, BLOCK)
    amax = blocks.abs().amax(dim=2).to(torch.float32)           # [M, K/128]
    sa = amax / 448.0
    Aq = (blocks.to(torch.float32) / sa[:, :, None]).to(torch.float8_e4m3fn)
    zero = amax == 0
    if bool(zero.any()):
        Aq.view(torch.uint8)[zero] = 0xFF
    return (Aq.reshape(M, K), sa.t().contiguous())
