"""Every output of the full-size GEMM configurations, not a row sample.

At these sizes the CPU oracle takes minutes per product, so the parity tests in
test_gpu_parity.py check it on sampled rows.  Here a plain PyTorch reference of
the same operation runs on the GPU in fp32 (fp64 where the tolerance asks for
it) and every output of the hip kernel is compared with it.  Each reference is
first pinned to the oracle on a row sample (the int4 dequantisation bit for
bit over the whole weight matrix), so what is checked everywhere is still the
oracle's arithmetic:

* W4A16 prefill (config 1 at M = 4096, and the 192-row tail shape), the
  grouped GEMM (config 4, every expert): fp16 within 1e-2 (the operator's
  tolerance), against fp16(A @ dequant(W)) accumulated in fp32;
* fp8 scaled GEMM (config 2, 8192^3): bf16 within 1e-2;
* matmul at K = 20480: fp16 within 2e-3, fp32 (three bf16 products) within
  1e-4 of the fp64 product, fp8 codes equal on > 99.5 % and never more than
  one e4m3 step apart; matmul_int8 bit for bit (fp64 sums of these integers
  are exact).
"""
import numpy as np
import pytest
import torch

import oracle
from tilebench_amd.data import tensors as T

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu case]", *a, flush=True)


@pytest.fixture
def fp32_matmul():
    """torch's fp32 matmul without TF32-style reduced-precision inputs."""
    old = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
    torch.backends.cuda.matmul.allow_tf32 = old


def _dequant_int4(p, s, z, G):
    """fp16 [K, N] = fp16((q - z) * s) on the device: codes from the low then high
    nibble of each byte (even, odd column), groups of G rows along K."""
    K, N = p.shape[0], p.shape[1] * 2
    q = torch.stack((p & 15, p >> 4), dim=-1).reshape(K, N).to(torch.int16)
    zz = torch.stack((z & 15, z >> 4), dim=-1).reshape(K // G, N).to(torch.int16)
    d = (q.view(K // G, G, N) - zz[:, None, :]).to(torch.float32) * s.to(torch.float32)[:, None, :]
    return d.to(torch.float16).reshape(K, N)


def _rows(M, n, seed):
    return np.sort(np.random.default_rng(seed).choice(M, min(M, n), replace=False))


def _allclose_everywhere(got, ref, tol, what):
    g, r = got.float(), ref.float()
    ok = torch.isclose(g, r, atol=tol, rtol=tol)
    bad = int((~ok).sum())
    same = float((got.view(torch.int16) == ref.view(torch.int16)).float().mean()) if got.element_size() == 2 else None
    print(f"  {what}: {got.numel()} outputs, max |diff| {float((g - r).abs().max()):.3g}, "
          f"bit-identical {same}, outside {tol}: {bad}", flush=True)
    assert bad == 0


@pytest.mark.parametrize("M,K,N,G", [(4096, 4096, 11008, 128), (3000, 512, 11008, 128)])
def test_w4a16_prefill_every_output(gpu, fp32_matmul, M, K, N, G):
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip

    _say("w4a16 prefill, every output", M, K, N, G)
    A, p, s, z, G = T.generate_w4a16_gemm_inputs(M, K, N, G, seed=1, device="cpu")
    Ag, pg, sg, zg = A.to(gpu), p.to(gpu), s.to(gpu), z.to(gpu)
    Wd = _dequant_int4(pg, sg, zg, G)
    # pin: the device dequantisation is the oracle's, bit for bit, over all of W
    Wo = oracle.int4_dequant(p.numpy(), s.numpy(), z.numpy(), G)
    assert np.array_equal(Wd.cpu().numpy().view(np.uint16), Wo.view(np.uint16))
    ref32 = Ag.float() @ Wd.float()
    # pin: the fp32 product rows equal the oracle's fp32 product on a sample
    rows = _rows(M, 16, 7)
    o32 = A.numpy()[rows].astype(np.float32) @ Wo.astype(np.float32)
    np.testing.assert_allclose(ref32[torch.as_tensor(rows, device=gpu)].cpu().numpy(), o32, rtol=1e-4,
                               atol=1e-4 * float(np.abs(o32).max()))
    Y = impl_hip.run(Ag, pg, sg, zg, G)
    torch.cuda.synchronize()
    _allclose_everywhere(Y, ref32.half(), 1e-2, "w4a16 prefill")


def test_grouped_gemm_every_output(gpu, fp32_matmul):
    """Config 4 (64 experts, 16384 tokens x top-8, Zipf 1.1): every row of every
    expert, padding rows included (they are zero rows of A, so zero outputs)."""
    from tilebench_amd.benchmarks.operators.moe_w4a16_grouped_gemm import impl_hip

    _say("grouped config 4, every output")
    A, p, s, z, off, G = T.generate_moe_w4a16_grouped_gemm_inputs(16384, 8, 64, 4096, 1408, 128, seed=4,
                                                                  device="cpu")
    Ag, pg, sg, zg, og = A.to(gpu), p.to(gpu), s.to(gpu), z.to(gpu), off.to(gpu)
    Y = impl_hip.run(Ag, pg, sg, zg, og, G)
    torch.cuda.synchronize()
    o = off.tolist()
    ref = torch.empty_like(Y)
    for e in range(64):
        lo, hi = o[e], o[e + 1]
        if hi > lo:
            ref[lo:hi] = (Ag[lo:hi].float() @ _dequant_int4(pg[e], sg[e], zg[e], G).float()).half()
    # pin: one expert's reference rows against the oracle
    e = int(np.argmax(np.diff(o)))
    rows = o[e] + _rows(o[e + 1] - o[e], 8, 3)
    want = oracle.w4a16_gemm(A.numpy()[rows], p.numpy()[e], s.numpy()[e], z.numpy()[e], G)
    np.testing.assert_allclose(ref[torch.as_tensor(rows, device=gpu)].cpu().numpy().astype(np.float32),
                               want.astype(np.float32), atol=1e-2, rtol=1e-2)
    _allclose_everywhere(Y, ref, 1e-2, "grouped")


def test_fp8_scaled_gemm_every_output(gpu, fp32_matmul):
    """Config 2 (8192^3): bf16(sa * sw * sum e4m3 * e4m3) everywhere."""
    from tilebench_amd.benchmarks.operators.fp8_scaled_gemm import impl_hip

    M = N = K = 8192
    _say("fp8_scaled_gemm, every output", M, N, K)
    Aq, Wq, sa, sw = T.generate_fp8_scaled_gemm_inputs(M, N, K, seed=2, device="cpu")
    Ag, Wg, sag, swg = Aq.to(gpu), Wq.to(gpu), sa.to(gpu), sw.to(gpu)
    Y = impl_hip.run(Ag, Wg, sag, swg)
    torch.cuda.synchronize()
    ref = ((Ag.float() @ Wg.float()) * sag[:, None] * swg[None, :]).to(torch.bfloat16)
    rows = _rows(M, 8, 5)
    want = oracle.bf16_bits_to_f32(oracle.fp8_scaled_gemm(Aq.view(torch.uint8).numpy()[rows],
                                                          Wq.contiguous().view(torch.uint8).numpy(),
                                                          sa.numpy()[rows], sw.numpy()))
    np.testing.assert_allclose(ref[torch.as_tensor(rows, device=gpu)].float().cpu().numpy(), want, atol=1e-2,
                               rtol=1e-2)
    _allclose_everywhere(Y, ref, 1e-2, "fp8 scaled GEMM")


def test_matmul_fp16_every_output(gpu, fp32_matmul):
    from tilebench_amd.benchmarks.operators.matmul_fp32_fp16_fp8 import impl_hip

    M, N, K = 4096, 4096, 20480
    _say("matmul fp16, every output", M, N, K)
    a, b = T.generate_matmul_fp32_fp16_fp8_inputs(M, N, K, dtype=torch.float16, seed=M + K, device="cpu")
    ag, bg = a.to(gpu), b.to(gpu)
    out = impl_hip.run(ag, bg)
    torch.cuda.synchronize()
    ref = (ag.float() @ bg.float()).half()
    rows = _rows(M, 8, 11)
    np.testing.assert_allclose(ref[torch.as_tensor(rows, device=gpu)].float().cpu().numpy(),
                               oracle.matmul_f16(a.numpy()[rows], b.numpy()).astype(np.float32), atol=2e-3, rtol=2e-3)
    _allclose_everywhere(out, ref, 2e-3, "matmul fp16")


def test_matmul_fp32_every_output(gpu):
    from tilebench_amd.benchmarks.operators.matmul_fp32_fp16_fp8 import impl_hip

    M, N, K = 4096, 4096, 20480
    _say("matmul fp32, every output", M, N, K)
    a, b = T.generate_matmul_fp32_fp16_fp8_inputs(M, N, K, dtype=torch.float32, seed=M + K, device="cpu")
    ag, bg = a.to(gpu), b.to(gpu)
    out = impl_hip.run(ag, bg)
    torch.cuda.synchronize()
    ref = (ag.double() @ bg.double()).float()
    rows = _rows(M, 8, 12)
    want = oracle.matmul_f32(a.numpy()[rows], b.numpy())
    # both are fp64 sums rounded once to fp32; their summation orders differ
    np.testing.assert_allclose(ref[torch.as_tensor(rows, device=gpu)].cpu().numpy(), want, rtol=1e-6,
                               atol=1e-6 * float(np.abs(want).max()))
    ok = torch.isclose(out, ref, atol=1e-4, rtol=1e-4)
    print(f"  matmul fp32: max |diff| {float((out - ref).abs().max()):.3g}, outside 1e-4: {int((~ok).sum())}",
          flush=True)
    assert bool(ok.all())


def test_matmul_fp8_every_output(gpu, fp32_matmul):
    from tilebench_amd.benchmarks.operators.matmul_fp32_fp16_fp8 import impl_hip

    M, N, K = 4096, 4096, 20480
    _say("matmul fp8, every output", M, N, K)
    a, b = T.generate_matmul_fp32_fp16_fp8_inputs(M, N, K, dtype=torch.float8_e4m3fn, seed=M + K, device="cpu")
    ag, bg = a.to(gpu), b.to(gpu)
    out = impl_hip.run(ag, bg).view(torch.uint8)
    torch.cuda.synchronize()
    ref = (ag.float() @ bg.float()).to(torch.bfloat16).float().to(torch.float8_e4m3fn).view(torch.uint8)
    rows = _rows(M, 8, 13)
    want = oracle.matmul_fp8(a.view(torch.uint8).numpy()[rows], b.view(torch.uint8).numpy())
    assert (ref[torch.as_tensor(rows, device=gpu)].cpu().numpy() == want).mean() > 0.995
    same = float((out == ref).float().mean())
    g = out.view(torch.float8_e4m3fn).float()
    r = ref.view(torch.float8_e4m3fn).float()
    step = torch.exp2(torch.floor(torch.log2(torch.clamp(r.abs(), min=2.0 ** -6))) - 3)
    far = int(((g - r).abs() > step + 1e-12).sum())
    print(f"  matmul fp8: codes equal {same:.5f}, more than one e4m3 step apart: {far}", flush=True)
    assert same > 0.995 and far == 0


def test_matmul_int8_every_output(gpu):
    from tilebench_amd.benchmarks.operators.matmul_int8 import impl_hip

    M, N, K = 2048, 2048, 20480
    _say("matmul_int8, every output", M, N, K)
    a, b = T.generate_matmul_int8_inputs(M, N, K, seed=M + K, device="cpu")
    ag, bg = a.to(gpu), b.to(gpu)
    out = impl_hip.run(ag, bg)
    torch.cuda.synchronize()
    B = torch.cat([((bg >> (2 * i)) & 3).to(torch.float64) - 1.0 for i in range(4)], dim=0)  # [K, N]
    ref = torch.round(ag.double() @ B).to(torch.int32)
    rows = _rows(M, 8, 14)
    np.testing.assert_array_equal(ref[torch.as_tensor(rows, device=gpu)].cpu().numpy(),
                                  oracle.matmul_int8(a.numpy()[rows], b.numpy()))
    assert torch.equal(out, ref)
