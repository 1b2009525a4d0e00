"""PyTorch reference of MoE top-k gating.

The reference operator (moe_topk_gating/impl_torch.py:4-20) takes
torch.topk(sorted=True) and a softmax over the k values in fp32, cast back to the
logits dtype, with int32 indices.  torch.topk does not order equal values by
index on the CPU, so the selection here is a stable descending sort: equal
logits keep ascending expert order (the BASELINE tie rule).  -0.0 and +0.0
compare equal and NaN ranks above every number, as in torch.sort/topk.
"""
import torch


def run(logits: torch.Tensor, M: int, E: int, k: int, **kwargs):
    vals, idx = torch.sort(logits, dim=-1, descending=True, stable=True)
    vals, idx = vals[:, :k], idx[:, :k]
    weights = torch.softmax(vals.to(torch.float32), dim=-1).to(logits.dtype)
    return (weights, idx.to(torch.int32))
