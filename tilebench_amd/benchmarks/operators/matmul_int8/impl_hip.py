"""hip backend of matmul_int8: tb_matmul_int8 in libtbhip.so (2-bit unpack into
a transposed int8 operand, then the int8 MFMA GEMM; exact int32 result)."""
import torch

from tilebench_amd import runtime as rt

rt.load_library()


def run(a: torch.Tensor, b: torch.Tensor, **kwargs):
    rt.require_device(a, b)
    if a.dtype != torch.int8 or b.dtype != torch.uint8:
        raise TypeError("matmul_int8 expects int8 a and uint8 b")
    a, b = a.contiguous(), b.contiguous()
    M, K = a.shape
    N = b.shape[1]
    if K != 4 * b.shape[0]:
        raise ValueError("A's K dim must be 4x B's K_b dim")
    out = torch.empty((M, N), dtype=torch.int32, device=a.device)
    need = rt.matmul_workspace_size(3, M, N, K)
    ws = torch.empty(need, dtype=torch.uint8, device=a.device)
    rt.call("tb_matmul_int8", a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K, ws.data_ptr(), need,
            rt.stream_handle(a.device))
    global _last_config
    _last_config = _config(M, N, K)
    return out


def _config(M, N, K):
    """The kernel choice of tb_matmul_int8 (nt_gemm.hip: big_tiles, int8_splits)."""
    tiles256 = -(-M // 256) * -(-N // 256)
    if tiles256 >= 256:
        return {"kernel": "nt_gemm<i8>", "tile": "256x256", "k_splits": 1}
    splits = min(8, 256 // tiles256, K // 128 // 8)
    if splits >= 2:
        return {"kernel": "nt_gemm<i8>", "tile": "256x256", "k_splits": splits}
    return {"kernel": "nt_gemm<i8>", "tile": "128x128", "k_splits": 1}


_last_config = None


def get_last_config():
    return _last_config
