"""Block-scaled fp8 on the GPU against the CPU oracle: the per-token,
per-128-channel activation quantiser (codes and scales bit for bit) and the
block-scaled GEMM (bf16 within the operator's 1e-2), including ragged M and N,
one K block, scales that vary over K, a full 8192^3 product checked on every
output against a GPU fp32 reference pinned to the oracle, and the reduction
to the row/column-scaled GEMM when the scales do not vary over K."""
import numpy as np
import pytest
import torch

import oracle
from tilebench_amd.data import tensors as T

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu case]", *a, flush=True)


def _u8(t):
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


@pytest.mark.parametrize("M,K", [(1, 128), (3, 384), (1000, 1024), (2048, 8192), (7, 7168)])
def test_fp8_act_quant_blocks_matches_oracle(gpu, M, K):
    from tilebench_amd.benchmarks.operators.fp8_act_quant_blocks import impl_hip

    _say("fp8_act_quant_blocks", M, K)
    (A,) = T.generate_fp8_act_quant_blocks_inputs(M, K, seed=M + K, device="cpu")
    Aq, sa = impl_hip.run(A.to(gpu))
    torch.cuda.synchronize()
    codes, s = oracle.fp8_act_quant_blocks(A.numpy())
    assert tuple(sa.shape) == (K // 128, M)
    np.testing.assert_array_equal(_u8(Aq), codes)
    np.testing.assert_array_equal(sa.cpu().numpy().view(np.uint32), s.view(np.uint32))


def test_fp8_act_quant_blocks_special_blocks(gpu):
    """Zero blocks (sa = 0, 0xFF codes), blocks holding inf or NaN (the integer
    encoder path), an exact 448 maximum, subnormal fp16 values and signed zeros,
    next to ordinary blocks of the same rows."""
    from tilebench_amd.benchmarks.operators.fp8_act_quant_blocks import impl_hip

    _say("fp8_act_quant_blocks special blocks")
    rng = np.random.default_rng(5)
    A = rng.standard_normal((6, 512)).astype(np.float16)
    A[0, :128] = 0
    A[1, 128:256] = 0
    A[1, 130] = np.float16(-0.0)
    A[2, 5] = np.inf
    A[3, 300] = np.nan
    A[3, 301] = np.uint16(0xFE00).view(np.float16)      # NaN with the sign bit set
    A[2, 6] = -np.inf
    A[4, 256:384] = np.float16(448.0) * np.sign(A[4, 256:384])
    A[5, 384:] = (rng.standard_normal(128) * 1e-6).astype(np.float16)   # subnormal fp16 values
    Aq, sa = impl_hip.run(torch.from_numpy(A).to(gpu))
    torch.cuda.synchronize()
    codes, s = oracle.fp8_act_quant_blocks(A)
    np.testing.assert_array_equal(_u8(Aq), codes)
    np.testing.assert_array_equal(sa.cpu().numpy().view(np.uint32), s.view(np.uint32))


def _block_check(gpu, M, N, K, seed, rows=None):
    from tilebench_amd.benchmarks.operators.fp8_block_scaled_gemm import impl_hip

    _say("fp8_block_scaled_gemm", M, N, K)
    Aq, WqT, sa, sw = T.generate_fp8_block_scaled_gemm_inputs(M, N, K, seed=seed, device="cpu")
    Y = impl_hip.run(Aq.to(gpu), WqT.to(gpu), sa.to(gpu), sw.to(gpu))
    torch.cuda.synchronize()
    got = Y.float().cpu().numpy()
    r = np.arange(M) if rows is None else rows
    ref = oracle.bf16_bits_to_f32(oracle.fp8_block_gemm(_u8(Aq)[r], _u8(WqT), sa.numpy()[:, r], sw.numpy()))
    np.testing.assert_allclose(got[r], ref, atol=1e-2, rtol=1e-2)
    assert np.isfinite(got).all()
    return got


@pytest.mark.parametrize("M,N,K", [(256, 128, 128), (256, 256, 256), (300, 200, 384), (1, 8, 128),
                                   (513, 1032, 1024), (64, 136, 2048), (1024, 1024, 4096)])
def test_fp8_block_gemm_matches_oracle(gpu, M, N, K):
    _block_check(gpu, M, N, K, seed=M + N + K)


def test_fp8_block_gemm_deepseek_shape_rows(gpu):
    """A DeepSeek-V3 projection shape (4096 tokens, N = 2112, K = 7168), rows sampled."""
    rows = np.sort(np.random.default_rng(3).choice(4096, 48, replace=False))
    _block_check(gpu, 4096, 2112, 7168, seed=9, rows=rows)


def test_fp8_block_gemm_repeat_is_bit_identical(gpu):
    from tilebench_amd.benchmarks.operators.fp8_block_scaled_gemm import impl_hip

    _say("fp8_block_scaled_gemm repeat")
    x = [t.to(gpu) for t in T.generate_fp8_block_scaled_gemm_inputs(512, 384, 1024, seed=4, device="cpu")]
    ys = [impl_hip.run(*x) for _ in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(ys[0], ys[1]) and torch.equal(ys[0], ys[2])


def test_fp8_block_gemm_uniform_scales_equal_row_column_gemm(gpu):
    """sa[kb, m] = r[m] and sw[nb, kb] = c[nb] for every block: the block GEMM
    and tb_fp8_scaled_gemm (sw[n] = c[n // 128]) agree to one bf16 step."""
    from tilebench_amd.benchmarks.operators.fp8_block_scaled_gemm import impl_hip as blk
    from tilebench_amd.benchmarks.operators.fp8_scaled_gemm import impl_hip as rowcol

    _say("fp8_block_scaled_gemm uniform scales")
    M, N, K = 512, 384, 1024
    Aq, WqT, _, _ = T.generate_fp8_block_scaled_gemm_inputs(M, N, K, seed=6, device="cpu")
    g = torch.Generator().manual_seed(6)
    r = torch.rand(M, generator=g) + 0.5
    c = torch.rand(3, generator=g) * 0.01 + 1e-3
    y_blk = blk.run(Aq.to(gpu), WqT.to(gpu), r.repeat(K // 128, 1).to(gpu), c[:, None].repeat(1, K // 128).to(gpu))
    y_rc = rowcol.run(Aq.to(gpu), WqT.to(gpu).t(), r.to(gpu), c.repeat_interleave(128)[:N].to(gpu))
    torch.cuda.synchronize()
    np.testing.assert_allclose(y_blk.float().cpu().numpy(), y_rc.float().cpu().numpy(), rtol=2 ** -7, atol=1e-30)


def test_fp8_block_gemm_full_size_every_output(gpu):
    """8192^3: every output against a GPU fp32 reference (the operands
    dequantised by the block map, one fp32 matmul), which is first pinned to
    the oracle on 32 rows; rows sampled against the oracle directly."""
    from tilebench_amd.benchmarks.operators.fp8_block_scaled_gemm import impl_hip, impl_torch

    M = N = K = 8192
    _say("fp8_block_scaled_gemm full", M, N, K)
    x = T.generate_fp8_block_scaled_gemm_inputs(M, N, K, seed=2, device="cpu")
    d = [t.to(gpu) for t in x]
    Y = impl_hip.run(*d)
    old = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        R = impl_torch.run(*d)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = old
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(8).choice(M, 32, replace=False))
    ref = oracle.bf16_bits_to_f32(oracle.fp8_block_gemm(_u8(x[0])[rows], _u8(x[1]), x[2].numpy()[:, rows],
                                                        x[3].numpy()))
    np.testing.assert_allclose(R.float().cpu().numpy()[rows], ref, atol=1e-2, rtol=1e-2)
    np.testing.assert_allclose(Y.float().cpu().numpy()[rows], ref, atol=1e-2, rtol=1e-2)
    ok = torch.isclose(Y.float(), R.float(), atol=1e-2, rtol=1e-2)
    assert bool(ok.all()), f"{int((~ok).sum())} of {ok.numel()} outputs outside 1e-2"
