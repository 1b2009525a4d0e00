"""hip backend of MoE top-k gating: tb_moe_topk_gating in libtbhip.so."""
import torch

from tilebench_amd import runtime as rt

rt.load_library()

_DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
_last_config = None


def run(logits: torch.Tensor, M: int, E: int, k: int, **kwargs):
    global _last_config
    rt.require_device(logits)
    if logits.dtype not in _DTYPES:
        raise TypeError(f"moe_topk_gating: unsupported logits dtype {logits.dtype}")
    if tuple(logits.shape) != (M, E):
        raise ValueError(f"moe_topk_gating: logits shape {tuple(logits.shape)} != ({M}, {E})")
    logits = logits.contiguous()
    weights = torch.empty((M, k), dtype=logits.dtype, device=logits.device)
    indices = torch.empty((M, k), dtype=torch.int32, device=logits.device)
    rt.call("tb_moe_topk_gating", logits.data_ptr(), weights.data_ptr(), indices.data_ptr(), M, E, k,
            _DTYPES[logits.dtype], rt.stream_handle(logits.device))
    if E in (64, 128, 256) and 2 < k <= 8:  # the dispatch of tb_moe_topk_gating (moe_gating.hip)
        _last_config = {"kernel": "filter_kernel", "lanes_per_row": 16, "per_lane": E // 16, "block": 256}
    else:
        lpr = 1 if E <= 16 else 2 if E <= 32 else 4 if E <= 64 else 8 if E <= 128 else 16 if E <= 256 else \
            32 if E <= 512 else 64
        _last_config = {"kernel": "gating_kernel", "lanes_per_row": lpr, "per_lane": 16, "block": 256}
    return (weights, indices)


def get_last_config():
    return _last_config
