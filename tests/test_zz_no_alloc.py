"""tb_w4a16_gemm_noalloc (the entry point that allocates nothing) against
tb_w4a16_gemm with a caller workspace, through the C ABI: the same kernels run
on the same inputs, so outputs must be identical bit for bit, on two decode
calls in a row (the second smaller), then on a prefill shape."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from tilebench_amd import runtime as rt
from tilebench_amd.data import tensors as T

pytestmark = pytest.mark.gpu


def _call_pair(lib, gpu, M, K, N, G, seed):
    A, p, s, z, G = T.generate_w4a16_gemm_inputs(M, K, N, G, seed=seed, device="cpu")
    Ad, pd, sd, zd = (t.to(gpu) for t in (A, p, s, z))
    stream = torch.cuda.current_stream().cuda_stream
    need = ctypes.c_int64(0)
    assert lib.tb_w4a16_workspace_size(M, N, K, G, ctypes.byref(need)) == 0
    ws = torch.zeros(max(need.value, 256), dtype=torch.uint8, device=gpu)
    y_ws = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
    y_na = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
    st = lib.tb_w4a16_gemm(Ad.data_ptr(), pd.data_ptr(), sd.data_ptr(), zd.data_ptr(), y_ws.data_ptr(), M, N, K, G,
                           ws.data_ptr(), need.value, stream)
    rt.check(st, "tb_w4a16_gemm")
    st = lib.tb_w4a16_gemm_noalloc(Ad.data_ptr(), pd.data_ptr(), sd.data_ptr(), zd.data_ptr(), y_na.data_ptr(),
                                   M, N, K, G, stream)
    rt.check(st, "tb_w4a16_gemm_noalloc")
    torch.cuda.synchronize()
    return y_ws.cpu(), y_na.cpu(), (A, p, s, z, G)


def test_noalloc_equals_workspace_entry_point(gpu):
    lib = rt.load_library()
    K, N, G = 4096, 11008, 128
    for i, M in enumerate((16, 1)):           # the second call is smaller
        print(f"[gpu case] noalloc decode M={M} K={K} N={N}", flush=True)
        y_ws, y_na, (A, p, s, z, G) = _call_pair(lib, gpu, M, K, N, G, seed=40 + i)
        assert torch.equal(y_ws.view(torch.int16), y_na.view(torch.int16)), f"M={M}: outputs differ"
        ref = oracle.w4a16_gemm(A.numpy(), p.numpy(), s.numpy(), z.numpy(), G)
        np.testing.assert_allclose(y_na.numpy().astype(np.float32), ref.astype(np.float32), atol=1e-2, rtol=1e-2)
    print("[gpu case] noalloc ragged N=1000 M=7", flush=True)
    y_ws, y_na, _ = _call_pair(lib, gpu, 7, 1024, 1000, 128, seed=43)
    assert torch.equal(y_ws.view(torch.int16), y_na.view(torch.int16))
    print("[gpu case] noalloc prefill M=300", flush=True)
    y_ws, y_na, _ = _call_pair(lib, gpu, 300, 512, 512, 128, seed=44)
    assert torch.equal(y_ws.view(torch.int16), y_na.view(torch.int16))


def test_noalloc_replays_from_a_graph(gpu):
    """Captured into a graph (no allocation inside the capture from the
    library), replayed with eager calls between the replays."""
    lib = rt.load_library()
    M, K, N, G = 16, 4096, 11008, 128
    A, p, s, z, G = T.generate_w4a16_gemm_inputs(M, K, N, G, seed=45, device="cpu")
    Ad, pd, sd, zd = (t.to(gpu) for t in (A, p, s, z))
    ref = oracle.w4a16_gemm(A.numpy(), p.numpy(), s.numpy(), z.numpy(), G).astype(np.float32)
    y = torch.empty((M, N), dtype=torch.float16, device=gpu)
    y2 = torch.empty((M, N), dtype=torch.float16, device=gpu)

    def call(out):
        rt.check(lib.tb_w4a16_gemm_noalloc(Ad.data_ptr(), pd.data_ptr(), sd.data_ptr(), zd.data_ptr(), out.data_ptr(),
                                           M, N, K, G, torch.cuda.current_stream().cuda_stream),
                 "tb_w4a16_gemm_noalloc")
    call(y2)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(y)
    for i in range(3):
        print(f"[gpu case] noalloc graph replay {i}", flush=True)
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_allclose(y.cpu().numpy().astype(np.float32), ref, atol=1e-2, rtol=1e-2)
        assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
        call(y2)
        torch.cuda.synchronize()
