"""PyTorch reference of weight_dequant (tilebench/benchmarks/operators/weight_dequant/impl_torch.py:4-8):
Y[i, j] = X[i, j] * S[i // T, j // T], computed in the tensors' dtype."""
import torch


def run(X: torch.Tensor, S: torch.Tensor, M: int, N: int, TILE_SIZE: int, **kwargs):
    scale = S.repeat_interleave(TILE_SIZE, dim=0)[:M].repeat_interleave(TILE_SIZE, dim=1)[:, :N]
    return X * scale
