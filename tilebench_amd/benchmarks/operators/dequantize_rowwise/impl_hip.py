"""hip backend of dequantize_rowwise: tb_dequantize_rowwise in libtbhip.so."""
import torch

from tilebench_amd import runtime as rt

rt.load_library()


def run(x: torch.Tensor, state_x: torch.Tensor, **kwargs):
    rt.require_device(x, state_x)
    if x.dtype != torch.int8 or state_x.dtype != torch.float32:
        raise TypeError("dequantize_rowwise expects int8 x and fp32 state_x")
    x, state_x = x.contiguous(), state_x.contiguous()
    rows, cols = x.shape
    y = torch.empty((rows, cols), dtype=torch.float16, device=x.device)
    rt.call("tb_dequantize_rowwise", x.data_ptr(), state_x.data_ptr(), y.data_ptr(), rows, cols,
            rt.stream_handle(x.device))
    return y


def get_last_config():
    return {"kernel": "dequant_rowwise_vec", "elements_per_thread": 16}
