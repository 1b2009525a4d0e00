"""hip backend of the W4A16 GEMM: libtbhip.so's tb_w4a16_gemm family.

The weights arrive in one of two layouts, and `run` reads the one it is given;
it keeps no state between calls (no per-weight copy, no cache):

* packed uint8 [K, N/2] (BASELINE config 0's layout): M <= 16 runs the split-K
  decode (tb_w4a16_gemm with its workspace), larger M the MFMA prefill;
* the decode's slab layout, uint8 [N/64, K/32, 1024] (a weight format of its
  own, converted once at load by tilebench_amd.formats.w4a16_to_slabs, as a
  checkpoint converter would): M <= 16 runs the slab decode
  (tb_w4a16_gemm_slabs), one block per 64-column slab with no cross-block
  reduction.  The prefill does not read this layout; M > 16 is refused.

Ownership follows the reference's contract (inputs read-only, a fresh output
per call; tilebench/llm/v2/contracts/data/weight_dequant/contract.md:31).
"""
import ctypes

import torch

from tilebench_amd import runtime as rt
from tilebench_amd.formats import SLAB_COLS, SLAB_UNIT

rt.load_library()

_last_config = None


def slab_shape_ok(M: int, N: int, K: int, group: int) -> bool:
    """Whether the slab decode takes this shape (tb_w4a16_gemm_slabs' limits,
    within the operator's own group % 64 == 0)."""
    return 1 <= M <= 16 and N % 64 == 0 and group in (64, 128) and K in (1024, 2048, 4096) and K % (16 * group) == 0


def _weight_shape(packed: torch.Tensor, K: int):
    """(N, layout) of the weight operand."""
    if packed.dim() == 3:
        if packed.shape[2] != 1024 or packed.shape[1] * SLAB_UNIT != K:
            raise ValueError(f"w4a16_gemm: slab-layout weights {tuple(packed.shape)} do not match K = {K}")
        return packed.shape[0] * SLAB_COLS, "slabs"
    if packed.dim() == 2:
        if packed.shape[0] != K:
            raise ValueError(f"w4a16_gemm: packed weights {tuple(packed.shape)} do not match K = {K}")
        return packed.shape[1] * 2, "rows"
    raise ValueError(f"w4a16_gemm: packed weights must be [K, N/2] or slabs [N/64, K/32, 1024], "
                     f"got {tuple(packed.shape)}")


def run(A: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, group: int, **kwargs):
    """Y = A @ dequant(packed) in fp16 (fp32 accumulation)."""
    global _last_config
    rt.require_device(A, packed, scales, zeros)
    if A.dtype != torch.float16 or packed.dtype != torch.uint8 or zeros.dtype != torch.uint8 \
            or scales.dtype != torch.float16:
        raise TypeError("w4a16_gemm expects fp16 A/scales and uint8 packed weights/zeros")
    M, K = A.shape
    N, layout = _weight_shape(packed, K)
    if tuple(scales.shape) != (K // group, N) or tuple(zeros.shape) != (K // group, N // 2):
        raise ValueError("w4a16_gemm: weight / scale / zero shapes do not match A")
    A, scales, zeros, packed = A.contiguous(), scales.contiguous(), zeros.contiguous(), packed.contiguous()
    Y = torch.empty((M, N), dtype=torch.float16, device=A.device)
    stream = rt.stream_handle(A.device)
    if layout == "slabs":
        if not slab_shape_ok(M, N, K, group):
            raise ValueError(f"w4a16_gemm: the slab layout is a decode format (1 <= M <= 16, G in {{64, 128}}, "
                             f"K in {{1024, 2048, 4096}}, K % 16G == 0); got M={M} K={K} N={N} G={group}")
        rt.call("tb_w4a16_gemm_slabs", A.data_ptr(), packed.data_ptr(), scales.data_ptr(), zeros.data_ptr(),
                Y.data_ptr(), M, N, K, group, stream)
        _last_config = {"kernel": "w4a16_slab_decode", "layout": "slabs", "cols_per_block": 64, "waves": 16}
        return Y
    need = ctypes.c_int64(0)
    rt.call("tb_w4a16_workspace_size", M, N, K, group, ctypes.byref(need))
    ws = rt.workspace(need.value, A.device, stream)
    rt.call("tb_w4a16_gemm", A.data_ptr(), packed.data_ptr(), scales.data_ptr(), zeros.data_ptr(), Y.data_ptr(),
            M, N, K, group, rt.ptr(ws), need.value, stream)
    _last_config = ({"kernel": "w4a16_decode", "layout": "rows", "cols_per_block": 256,
                     "workspace_bytes": need.value}
                    if M <= 16 else {"kernel": "w4a16_prefill", "layout": "rows", "BM": 256, "BN": 256, "BK": 64})
    return Y


def get_last_config():
    return _last_config
