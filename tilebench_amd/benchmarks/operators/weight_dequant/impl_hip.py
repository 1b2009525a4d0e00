"""hip backend of weight_dequant: tb_weight_dequant in libtbhip.so."""
import torch

from tilebench_amd import runtime as rt

rt.load_library()

_DT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def run(X: torch.Tensor, S: torch.Tensor, M: int, N: int, TILE_SIZE: int, **kwargs):
    rt.require_device(X, S)
    if X.dtype not in _DT or S.dtype != X.dtype:
        raise TypeError(f"weight_dequant: unsupported dtypes {X.dtype} / {S.dtype}")
    X, S = X.contiguous(), S.contiguous()
    Y = torch.empty((M, N), dtype=X.dtype, device=X.device)
    rt.call("tb_weight_dequant", X.data_ptr(), S.data_ptr(), Y.data_ptr(), M, N, TILE_SIZE, _DT[X.dtype],
            rt.stream_handle(X.device))
    return Y


def get_last_config():
    return {"kernel": "weight_dequant_vec", "elements_per_thread": 8}
