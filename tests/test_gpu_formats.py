"""Converted checkpoints through the hip kernels: a GPTQ act-order layer and an
AWQ layer through the W4A16 GEMM (prefill and decode shapes), an e4m3fnuz fp8
layer through the scaled fp8 GEMM, each against the CPU oracle on the
converted operands and, for the int4 formats, against the format's own
definition computed in float64."""
import numpy as np
import pytest
import torch

import oracle
from tilebench_amd import formats as F

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu case]", *a, flush=True)


def _checkpoint_codes(K, N, G, seed):
    rng = np.random.default_rng(seed)
    q = torch.from_numpy(rng.integers(0, 16, size=(K, N), dtype=np.uint8))
    z = torch.from_numpy(rng.integers(0, 16, size=(K // G, N), dtype=np.uint8))
    s = torch.from_numpy((rng.random((K // G, N)) * 9e-3 + 1e-3).astype(np.float16))
    return q, z, s, rng


@pytest.mark.parametrize("M", [4, 300])
def test_gptq_act_order_layer(gpu, M):
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip

    K, N, G = 4096, 1024, 128
    _say("gptq act-order", M, K, N, G)
    q, z, s, rng = _checkpoint_codes(K, N, G, 80 + M)
    g_idx = torch.from_numpy((rng.permutation(K) // G).astype(np.int32))
    # a v1 checkpoint written through the inverse converter (its packing is
    # pinned against a bit-by-bit restatement of the format on the CPU)
    base = F.Int4Weights(F.pack_columns(q), s, F.pack_columns(z), G)
    qweight, qzeros, scales, _ = F.tb_to_gptq(base)
    w = F.gptq_to_tb(qweight, qzeros, scales, g_idx)
    A = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16))
    Ap = F.permute_input(A, w.perm)
    dev = [t.to(gpu) for t in (Ap, w.packed, w.scales, w.zeros)]
    Y = impl_hip.run(*dev, G)
    torch.cuda.synchronize()
    got = Y.cpu().numpy().astype(np.float32)
    want = oracle.w4a16_gemm(Ap.numpy(), w.packed.numpy(), w.scales.numpy(), w.zeros.numpy(), G).astype(np.float32)
    np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2)
    # the GPTQ definition on the original channel order: W[k] uses group g_idx[k]
    gi = g_idx.numpy().astype(np.int64)
    Wdef = (q.numpy().astype(np.float64) - z.numpy()[gi].astype(np.float64)) * s.numpy()[gi].astype(np.float64)
    ref = A.numpy().astype(np.float64) @ Wdef.astype(np.float16).astype(np.float64)
    np.testing.assert_allclose(got, ref, rtol=2e-2, atol=2e-2)


def test_awq_layer(gpu):
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip

    K, N, G, M = 2048, 512, 128, 256
    _say("awq", M, K, N, G)
    q, z, s, rng = _checkpoint_codes(K, N, G, 90)
    qweight, qzeros, scales = F.tb_to_awq(F.Int4Weights(F.pack_columns(q), s, F.pack_columns(z), G))
    w = F.awq_to_tb(qweight, qzeros, scales)
    A = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16))
    dev = [t.to(gpu) for t in (A, w.packed, w.scales, w.zeros)]
    Y = impl_hip.run(*dev, G)
    torch.cuda.synchronize()
    want = oracle.w4a16_gemm(A.numpy(), w.packed.numpy(), w.scales.numpy(), w.zeros.numpy(), G)
    np.testing.assert_allclose(Y.cpu().numpy().astype(np.float32), want.astype(np.float32), rtol=1e-2, atol=1e-2)


def test_fp8_fnuz_checkpoint_layer(gpu):
    from tilebench_amd.benchmarks.operators.fp8_scaled_gemm import impl_hip
    from tilebench_amd.benchmarks.operators.fp8_act_quant import impl_torch as quant_ref

    M, N, K = 256, 512, 1024
    _say("fp8 fnuz checkpoint", M, N, K)
    g = torch.Generator().manual_seed(95)
    Wf = torch.randn(N, K, generator=g) * 0.02
    amax = Wf.abs().amax(dim=1, keepdim=True)
    fnuz = (Wf / (amax / 240.0)).to(torch.float8_e4m3fnuz)          # an MI300-era checkpoint
    fw = F.fp8_checkpoint_to_tb(fnuz, amax / 240.0)
    Aq, sa = quant_ref.run(torch.randn(M, K, generator=g).to(torch.float16))
    Wq = fw.wqT.view(torch.float8_e4m3fn).t()
    dev = [t.to(gpu) for t in (Aq, Wq, sa, fw.sw)]
    Y = impl_hip.run(*dev)
    torch.cuda.synchronize()
    want = oracle.fp8_scaled_gemm(Aq.view(torch.uint8).numpy(), fw.wqT.numpy().T, sa.numpy(), fw.sw.numpy())
    got = Y.view(torch.int16).cpu().numpy().view(np.uint16)
    a, b = oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(want)
    np.testing.assert_allclose(a, b, rtol=1e-2, atol=1e-2)
