"""GPU parity of the MoE layer around config 4, step by step and end to end,
against the CPU oracle on the same seeded inputs.

Bit-exact: the expert sort (moe_align) and the combine (an in-order fp32 sum).
The GEMM steps compare fp16 outputs within rtol = atol = 1e-2 (the grouped
GEMM's tolerance), and also require most values to be bit-identical (only the
fp32 accumulation order differs).
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from tilebench_amd import runtime as rt
from tilebench_amd.data import tensors as T

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu case]", *a, flush=True)


def _np(t):
    return t.detach().cpu().numpy()


def _close(got, want, exact_frac=0.9, tol=1e-2):
    got = np.asarray(got, dtype=np.float16).astype(np.float32)
    want = np.asarray(want, dtype=np.float16).astype(np.float32)
    np.testing.assert_allclose(got, want, rtol=tol, atol=tol)
    frac = float((got == want).mean()) if got.size else 1.0
    assert frac >= exact_frac, frac


def _align(ids, E):
    P = ids.numel()
    sid = torch.full((P,), -7, dtype=torch.int32, device=ids.device)
    off = torch.full((E + 1,), -7, dtype=torch.int32, device=ids.device)
    rt.call("tb_moe_align", rt.ptr(ids), P, E, rt.ptr(sid), rt.ptr(off), rt.stream_handle(ids.device))
    torch.cuda.synchronize()
    return sid, off


@pytest.mark.parametrize("case", ["zipf16384x8of64", "invalid_ids_ragged", "misaligned", "one_expert", "e256"])
def test_moe_align_bit_exact(gpu, case):
    _say("moe_align", case)
    rng = np.random.default_rng(31)
    if case == "zipf16384x8of64":
        ids, E = T.zipf_routing(16384, 8, 64, 1.1, seed=4).to(torch.int32), 64
    elif case == "invalid_ids_ragged":
        ids, E = torch.from_numpy(rng.integers(-3, 9, size=(1001, 3)).astype(np.int32)), 6
    elif case == "misaligned":
        base = torch.from_numpy(rng.integers(0, 5, size=(4 * 777 + 1,)).astype(np.int32))
        ids, E = base, 5
    elif case == "one_expert":
        ids, E = torch.full((513, 2), 3, dtype=torch.int32), 4
    else:
        ids, E = T.zipf_routing(4096, 8, 256, 1.1, seed=5).to(torch.int32), 256
    dev = ids.to(gpu)
    if case == "misaligned":
        dev = dev[1:]                        # 4-byte aligned, not 16: the scalar load path
        ids = ids[1:]
    sid, off = _align(dev.contiguous() if case != "misaligned" else dev, E)
    want_sid, want_off = oracle.moe_align(ids.numpy(), E)
    n = len(want_sid)
    np.testing.assert_array_equal(_np(off), want_off)
    np.testing.assert_array_equal(_np(sid)[:n], want_sid)
    assert (_np(sid)[n:] == -7).all()        # nothing written past the routed pairs


def _weights(E, H, I, g13, g2, seed):
    g = T._gen(seed)
    return T.random_int4_weights(H, 2 * I, g13, g, experts=E) + T.random_int4_weights(I, H, g2, g, experts=E)


@pytest.mark.parametrize("Tk,E,k,H,I,g13", [(300, 6, 2, 256, 192, 64), (97, 3, 3, 512, 128, 128),
                                             (1024, 64, 8, 4096, 704, 128)])
def test_gate_up_matches_oracle(gpu, Tk, E, k, H, I, g13):
    _say("moe_gate_up", Tk, E, k, H, I, g13)
    g = T._gen(40 + Tk)
    X = torch.randn(Tk, H, generator=g).to(torch.float16)
    ids = T.zipf_routing(Tk, k, E, 1.1, seed=41).to(torch.int32)
    W13, S13, Z13, *_ = _weights(E, H, I, g13, 64, 42)
    assert W13.shape == (E, H, I) and S13.shape == (E, H // g13, 2 * I) and Z13.shape == (E, H // g13, I)
    sid_np, off_np = oracle.moe_align(ids.numpy(), E)
    P = Tk * k
    sid, off = torch.from_numpy(sid_np).to(gpu), torch.from_numpy(off_np).to(gpu)
    assert off_np[-1] == len(sid_np) <= P and X.shape == (Tk, H)
    act = torch.empty((P, I), dtype=torch.float16, device=gpu)
    Xd, Wd, Sd, Zd = X.to(gpu), W13.to(gpu), S13.to(gpu), Z13.to(gpu)
    rt.call("tb_moe_w4a16_gate_up", rt.ptr(Xd), rt.ptr(sid), rt.ptr(off), rt.ptr(Wd), rt.ptr(Sd), rt.ptr(Zd),
            rt.ptr(act), Tk, k, E, H, I, g13, rt.stream_handle(gpu))
    torch.cuda.synchronize()
    want = oracle.moe_gate_up(X.numpy(), sid_np, off_np, k, W13.numpy(), S13.numpy(), Z13.numpy(), g13)
    _close(_np(act), want)


@pytest.mark.parametrize("Tk,E,k,I,H,g2", [(300, 6, 2, 192, 256, 64), (1024, 64, 8, 704, 4096, 64)])
def test_down_matches_oracle_and_leaves_unrouted_rows(gpu, Tk, E, k, I, H, g2):
    _say("moe_down", Tk, E, k, I, H, g2)
    g = T._gen(50 + Tk)
    ids = T.zipf_routing(Tk, k, E, 1.1, seed=51).to(torch.int32)
    ids[::7, 0] = E + 3                       # some pairs routed nowhere
    w = torch.rand(Tk, k, generator=g).to(torch.float32)
    act = (torch.randn(Tk * k, I, generator=g) * 2).to(torch.float16)
    *_, W2, S2, Z2 = _weights(E, H, I, 64, g2, 52)
    assert W2.shape == (E, I, H // 2) and S2.shape == (E, I // g2, H) and Z2.shape == (E, I // g2, H // 2)
    sid_np, off_np = oracle.moe_align(ids.numpy(), E)
    n = len(sid_np)
    act_sorted = act[:n]                      # rows in sorted order (any values)
    P = Tk * k
    assert off_np[-1] == n <= P and act_sorted.shape == (n, I) and w.numel() == P
    y = torch.full((P, H), float("nan"), dtype=torch.float16, device=gpu)
    # every device buffer stays referenced until the kernel has finished
    dev = [t.to(gpu) for t in (act_sorted, torch.from_numpy(sid_np), torch.from_numpy(off_np), w, W2, S2, Z2)]
    rt.call("tb_moe_w4a16_down", *[rt.ptr(t) for t in dev], rt.ptr(y), P, E, I, H, g2, rt.stream_handle(gpu))
    torch.cuda.synchronize()
    want, written = oracle.moe_down(act_sorted.numpy(), sid_np, off_np, w.numpy(), P, W2.numpy(), S2.numpy(),
                                    Z2.numpy(), g2)
    got = _np(y)
    _close(got[written], want[written])
    assert np.isnan(got[~written].astype(np.float32)).all()


def test_combine_bit_exact(gpu):
    _say("moe_combine")
    g = T._gen(60)
    Tk, k, E, H = 1000, 8, 64, 4096
    y = torch.randn(Tk * k, H, generator=g).to(torch.float16)
    assert y.shape == (Tk * k, H)
    ids = T.zipf_routing(Tk, k, E, 1.1, seed=61).to(torch.int32)
    ids[5, 3] = -1
    ids[17, 0] = E
    out = torch.empty((Tk, H), dtype=torch.float16, device=gpu)
    yd, idsd = y.to(gpu), ids.to(gpu)
    rt.call("tb_moe_combine", rt.ptr(yd), rt.ptr(idsd), rt.ptr(out), Tk, k, E, H, rt.stream_handle(gpu))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_np(out).view(np.uint16), oracle.moe_combine(y.numpy(), ids.numpy(), E).view(np.uint16))


def _layer_inputs(tokens, E=64, k=8, H=4096, I=704, seed=15):
    return T.generate_fused_moe_w4a16_inputs(tokens, E, k, H, I, 128, 64, seed=seed, device="cpu")


@pytest.mark.parametrize("tokens,E,k,H,I", [(64, 8, 2, 256, 128), (512, 64, 8, 4096, 704), (16384, 64, 8, 4096, 704)])
def test_fused_layer_matches_oracle(gpu, tokens, E, k, H, I):
    from tilebench_amd.benchmarks.operators.fused_moe_w4a16 import impl_hip

    _say("fused_moe_w4a16", tokens, E, k, H, I)
    inp = T.generate_fused_moe_w4a16_inputs(tokens, E, k, H, I, 128, 64, seed=15 + tokens, device="cpu")
    out = impl_hip.run(*[t.to(gpu) if torch.is_tensor(t) else t for t in inp])
    torch.cuda.synchronize()
    want = oracle.fused_moe_w4a16(*[t.numpy() if torch.is_tensor(t) else t for t in inp])
    _close(_np(out), want, exact_frac=0.8)


def test_fused_layer_is_deterministic_and_graph_replays_match(gpu):
    from tilebench_amd.benchmarks.operators.fused_moe_w4a16 import impl_hip

    _say("fused_moe_w4a16 determinism + graph")
    inp = [t.to(gpu) if torch.is_tensor(t) else t for t in _layer_inputs(2048, seed=70)]
    a = impl_hip.run(*inp)
    b = impl_hip.run(*inp)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        impl_hip.run(*inp)                    # warm the allocator on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        c = impl_hip.run(*inp)
    for _ in range(3):
        c.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(c.view(torch.int16), a.view(torch.int16))
        impl_hip.run(*inp)                    # eager work between replays
        torch.cuda.synchronize()


def test_fused_layer_rejects_bad_shapes_before_launching(gpu):
    lib = rt.load_library()
    need = ctypes.c_int64(0)
    rt.call("tb_fused_moe_w4a16_workspace_size", 16, 2, 4, 256, 96, ctypes.byref(need))
    ws = torch.empty(need.value, dtype=torch.uint8, device=gpu)
    X = torch.zeros(16, 256, dtype=torch.float16, device=gpu)
    L = torch.zeros(16, 4, dtype=torch.float32, device=gpu)
    dummy = torch.zeros(1 << 16, dtype=torch.uint8, device=gpu)
    with pytest.raises(ValueError, match="multiples of 64"):
        rt.call("tb_fused_moe_w4a16", rt.ptr(X), rt.ptr(L), *[rt.ptr(dummy)] * 6, rt.ptr(X), 16, 4, 2, 256, 96, 128,
                64, rt.ptr(ws), need.value, rt.stream_handle(gpu))
    assert lib is not None
