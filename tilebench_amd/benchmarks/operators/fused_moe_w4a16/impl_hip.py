"""hip backend of the MoE layer: tb_fused_moe_w4a16 in libtbhip.so (gating,
align, gate/up + SiLU, down, combine; five launches on the current stream,
no host synchronisation, so a call can be captured into a graph)."""
import ctypes

import torch

from tilebench_amd import runtime as rt

rt.load_library()

_last_config = None


def workspace_size(tokens: int, topk: int, experts: int, H: int, I: int) -> int:
    out = ctypes.c_int64(0)
    rt.call("tb_fused_moe_w4a16_workspace_size", tokens, topk, experts, H, I, ctypes.byref(out))
    return out.value


def run(X, logits, W13, S13, Z13, W2, S2, Z2, topk: int, group13: int, group2: int, **kwargs):
    global _last_config
    rt.require_device(X, logits, W13, S13, Z13, W2, S2, Z2)
    if X.dtype != torch.float16 or logits.dtype != torch.float32:
        raise TypeError("fused_moe_w4a16 expects fp16 X and fp32 router logits")
    if any(t.dtype != torch.uint8 for t in (W13, Z13, W2, Z2)) or S13.dtype != torch.float16 \
            or S2.dtype != torch.float16:
        raise TypeError("fused_moe_w4a16 expects uint8 packed weights / zeros and fp16 scales")
    T, H = X.shape
    E = logits.shape[1]
    I = W13.shape[-1]
    if tuple(logits.shape) != (T, E) or tuple(W13.shape) != (E, H, I) \
            or tuple(S13.shape) != (E, H // group13, 2 * I) or tuple(Z13.shape) != (E, H // group13, I) \
            or tuple(W2.shape) != (E, I, H // 2) or tuple(S2.shape) != (E, I // group2, H) \
            or tuple(Z2.shape) != (E, I // group2, H // 2):
        raise ValueError("fused_moe_w4a16: logits / weight / scale / zero shapes do not match X")
    X, logits = X.contiguous(), logits.contiguous()
    W13, S13, Z13, W2, S2, Z2 = (t.contiguous() for t in (W13, S13, Z13, W2, S2, Z2))
    out = torch.empty((T, H), dtype=torch.float16, device=X.device)
    need = workspace_size(T, topk, E, H, I)
    ws = torch.empty(need, dtype=torch.uint8, device=X.device)
    rt.call("tb_fused_moe_w4a16", X.data_ptr(), logits.data_ptr(), W13.data_ptr(), S13.data_ptr(), Z13.data_ptr(),
            W2.data_ptr(), S2.data_ptr(), Z2.data_ptr(), out.data_ptr(), T, E, topk, H, I, group13, group2,
            rt.ptr(ws), need, rt.stream_handle(X.device))
    _last_config = {"kernels": ["gating", "moe_align", "moe_gate_up", "moe_down", "moe_combine"],
                    "BM": 256, "BN_gate_up": 128, "BN_down": 256, "workspace_bytes": need}
    return out


def get_last_config():
    return _last_config
