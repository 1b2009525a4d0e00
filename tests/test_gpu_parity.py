"""GPU parity of every hip kernel against the CPU oracle (seeded inputs).

Bit-exact for dequantised values, fp8 codes, fp32 scales and top-k indices;
gating weights within 1e-5.  Each case prints its name and shape before the GPU
call so that a failing run names its case.
"""
import numpy as np
import pytest
import torch

import oracle
from tilebench_amd import formats
from tilebench_amd.data import tensors as T

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu case]", *a, flush=True)


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


# ----------------------------------------------------------------------------- int4 dequant

@pytest.mark.parametrize("K,N,G", [(4096, 4096, 128), (256, 512, 128), (128, 32, 64), (64, 6, 32), (128, 4096, 32)])
def test_int4_dequant_matches_oracle(gpu, K, N, G):
    from tilebench_amd.benchmarks.operators.int4_dequant import impl_hip

    _say("int4_dequant", K, N, G)
    p, s, z, K, N, G = T.generate_int4_dequant_inputs(K, N, G, seed=K + N, device="cpu")
    out = impl_hip.run(p.to(gpu), s.to(gpu), z.to(gpu), K, N, G)
    torch.cuda.synchronize()
    ref = oracle.int4_dequant(p.numpy(), s.numpy(), z.numpy(), G)
    np.testing.assert_array_equal(_u16(out), ref.view(np.uint16))


def test_int4_dequant_exhaustive_codes(gpu):
    """Every (q, z) pair against every scale of a spread of fp16 scales (incl. negative and subnormal)."""
    from tilebench_amd.benchmarks.operators.int4_dequant import impl_hip

    _say("int4_dequant exhaustive")
    K, N, G = 256, 256, 16   # 16 groups; within a group rows cover q = 0..15
    q = np.tile(np.arange(16, dtype=np.uint8)[:, None], (K // 16, N))          # row r -> q = r % 16
    zc = np.tile(np.arange(16, dtype=np.uint8), (K // G, N // 16))              # col n -> z = n % 16
    rng = np.random.default_rng(7)
    sbits = rng.integers(0, 0x7C00, size=(K // G, N), dtype=np.uint16)          # every finite magnitude band
    sbits[rng.random((K // G, N)) < 0.5] |= 0x8000
    scales = sbits.view(np.float16)
    packed, zeros = oracle.pack_int4(q), oracle.pack_int4(zc)
    out = impl_hip.run(torch.from_numpy(packed).to(gpu), torch.from_numpy(scales.copy()).to(gpu),
                       torch.from_numpy(zeros).to(gpu), K, N, G)
    torch.cuda.synchronize()
    ref = oracle.int4_dequant(packed, scales, zeros, G)
    np.testing.assert_array_equal(_u16(out), ref.view(np.uint16))


# ----------------------------------------------------------------------------- gating

@pytest.mark.parametrize("M,E,k,dist", [(16384, 64, 8, "normal"), (16384, 256, 8, "normal"), (1000, 128, 2, "grid"),
                                        (333, 20, 5, "normal"), (64, 1024, 32, "normal"), (7, 8, 8, "normal"),
                                        (100, 512, 8, "normal"), (65, 100, 3, "normal")])
def test_gating_matches_oracle(gpu, M, E, k, dist):
    from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_hip

    _say("gating", M, E, k, dist)
    logits, M, E, k = T.generate_moe_topk_gating_inputs(M, E, k, dist=dist, seed=M + E, device="cpu")
    w, i = impl_hip.run(logits.to(gpu), M, E, k)
    torch.cuda.synchronize()
    rw, ri = oracle.moe_topk_gating(logits.numpy(), k)
    np.testing.assert_array_equal(i.cpu().numpy(), ri)
    np.testing.assert_allclose(w.cpu().numpy(), rw, atol=1e-5, rtol=1e-5)


def test_gating_ties_nan_signed_zero(gpu):
    from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_hip

    _say("gating ties")
    rng = np.random.default_rng(3)
    x = rng.integers(-3, 4, size=(512, 64)).astype(np.float32)   # heavy ties
    x[5, 10] = -0.0
    x[6, :] = 0.0
    x[6, 7] = -0.0
    x[7, 3] = np.nan
    x[8, :] = -np.inf
    x[9, 60] = np.inf
    w, i = impl_hip.run(torch.from_numpy(x).to(gpu), 512, 64, 8)
    torch.cuda.synchronize()
    rw, ri = oracle.moe_topk_gating(x, 8)
    np.testing.assert_array_equal(i.cpu().numpy(), ri)
    np.testing.assert_allclose(w.cpu().numpy(), rw, atol=1e-5, rtol=1e-5, equal_nan=True)


def _filter_rows(E):
    """Rows that steer the filter kernel (E = 16·V, 16 lanes per row, lane q
    owning elements c·64 + 4q + i in fp32) through both of its paths: the
    threshold T is the k-th largest lane maximum and the row's candidates are
    the elements >= T.  Results are checked against the oracle either way."""
    rng = np.random.default_rng(E)
    rows = []
    base = lambda: rng.uniform(-5, -1, E).astype(np.float32)
    r = base(); r[np.arange(16) * 4] = 1.0                 # 16 tied candidates: filter path
    rows.append(r)
    r = base(); r[np.arange(16) * 4] = 1.0; r[1] = 1.0     # 17 candidates: the two-list sort (17..32)
    rows.append(r)
    r = base(); r[np.arange(16) * 4] = 1.0; r[np.arange(16) * 4 + 1] = 1.0; r[2] = 1.0
    rows.append(r)                                           # 33 candidates: exact path for its wavefront
    r = base(); r[np.arange(16) * 4] = 0.0; r[8] = -0.0; r[2] = -0.0   # signed zeros at the threshold
    rows.append(r)
    r = base(); r[np.arange(8) * 8] = 2.0; r[np.arange(8) * 8 + 2] = 2.0  # ties inside lanes
    rows.append(r)
    r = rng.standard_normal(E).astype(np.float32); r[E // 3] = np.inf
    rows.append(r)
    r = rng.standard_normal(E).astype(np.float32); r[E - 1] = np.nan
    rows.append(r)
    r = rng.standard_normal(E).astype(np.float32); r[5] = -np.inf
    rows.append(r)
    r = np.full(E, 3.0, np.float32)                          # every element tied
    rows.append(r)
    # Candidates whose order keys differ only in their low five bits (the
    # candidate sort's short keys hold their list slots there): the larger
    # value at the higher index (short-key order wrong, the wavefront re-sorts
    # the exact pairs), at the lower index (short-key order right), and three
    # negative values of which the middle index is the largest.
    up = lambda v: np.nextafter(np.float32(v), np.float32(np.inf))
    r = rng.standard_normal(E).astype(np.float32); r[3] = 4.0; r[E - 5] = up(4.0)
    rows.append(r)
    r = rng.standard_normal(E).astype(np.float32); r[E - 5] = 4.0; r[3] = up(4.0)
    rows.append(r)
    r = base(); r[[1, 22, 43]] = -0.5; r[22] = up(-0.5)
    rows.append(r)
    return np.stack(rows)


@pytest.mark.parametrize("E", [64, 128, 256])
@pytest.mark.parametrize("k", [1, 2, 3, 7, 8])
def test_gating_filter_paths(gpu, E, k):
    """The filter kernel's shapes (E in {64, 128, 256}, k <= 8): random rows
    (filter path) mixed with rows that take its two-list sort (17 to 32
    candidates), rows that force the exact path for their wavefront (more
    than 32 candidates, inf, NaN), ties and signed zeros at the threshold, and
    a ragged row count."""
    from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_hip

    _say("gating filter paths", E, k)
    rng = np.random.default_rng(100 * E + k)
    x = rng.standard_normal((1001, E)).astype(np.float32)
    special = _filter_rows(E)
    x[17:17 + len(special)] = special            # in the wavefronts of rows 16..19 to 28..31
    x[600:600 + len(special)] = special[::-1]
    w, i = impl_hip.run(torch.from_numpy(x).to(gpu), x.shape[0], E, k)
    torch.cuda.synchronize()
    rw, ri = oracle.moe_topk_gating(x, k)
    np.testing.assert_array_equal(i.cpu().numpy(), ri)
    np.testing.assert_allclose(w.cpu().numpy(), rw, atol=1e-5, rtol=1e-5, equal_nan=True)


@pytest.mark.parametrize("E", [64, 128, 256])
def test_gating_filter_ragged_row_counts(gpu, E):
    """Row counts that leave part of the last block past M (whose lanes read
    zeros and must write nothing): every row equals the oracle, and the rows
    of a larger output buffer past M keep their contents."""
    from tilebench_amd import runtime as rt

    for M in (1, 15, 17, 33, 1009):
        _say("gating filter ragged", E, M)
        logits, M, E, k = T.generate_moe_topk_gating_inputs(M, E, 8, seed=M * E, device="cpu")
        x = logits.to(gpu)
        w = torch.full((M + 16, k), 7.0, device=gpu)
        i = torch.full((M + 16, k), -7, dtype=torch.int32, device=gpu)
        rt.call("tb_moe_topk_gating", x.data_ptr(), w.data_ptr(), i.data_ptr(), M, E, k, 0, rt.stream_handle())
        torch.cuda.synchronize()
        rw, ri = oracle.moe_topk_gating(logits.numpy(), k)
        np.testing.assert_array_equal(i[:M].cpu().numpy(), ri)
        np.testing.assert_allclose(w[:M].cpu().numpy(), rw, atol=1e-5, rtol=1e-5)
        assert bool((w[M:] == 7.0).all()) and bool((i[M:] == -7).all())


@pytest.mark.parametrize("E", [64, 256])
@pytest.mark.parametrize("dt", ["fp16", "bf16"])
def test_gating_filter_half_dtypes(gpu, E, dt):
    """fp16 / bf16 logits at the BASELINE shapes (k = 8): indices bit-exact;
    weights within one unit in the last place of the half type (the fp32
    softmax matches the oracle to ~1e-7, so a rounding to half may land one
    step away)."""
    from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_hip

    _say("gating filter", E, dt)
    tdt = torch.float16 if dt == "fp16" else torch.bfloat16
    logits, M, E, k = T.generate_moe_topk_gating_inputs(4099, E, 8, dtype=tdt, seed=E, device="cpu")
    special = torch.from_numpy(_filter_rows(E)).to(tdt)
    logits[40:40 + special.shape[0]] = special
    w, i = impl_hip.run(logits.to(gpu), M, E, k)
    torch.cuda.synchronize()
    bits = logits.view(torch.int16).numpy().view(np.uint16) if dt == "bf16" else logits.numpy()
    rw, ri = oracle.moe_topk_gating(bits, k, dtype=dt)
    np.testing.assert_array_equal(i.cpu().numpy(), ri)
    got = _u16(w).astype(np.int32)
    want = np.asarray(rw).view(np.uint16).astype(np.int32)
    nan = np.isnan(w.float().cpu().numpy())
    assert np.array_equal(nan, np.isnan(oracle.bf16_bits_to_f32(rw) if dt == "bf16" else rw.astype(np.float32)))
    assert np.abs(got - want)[~nan].max() <= 1


@pytest.mark.parametrize("dt", ["fp16", "bf16"])
def test_gating_half_dtypes(gpu, dt):
    from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_hip
    from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_torch

    _say("gating", dt)
    tdt = torch.float16 if dt == "fp16" else torch.bfloat16
    logits, M, E, k = T.generate_moe_topk_gating_inputs(2048, 128, 2, dtype=tdt, dist="grid", seed=11, device="cpu")
    w, i = impl_hip.run(logits.to(gpu), M, E, k)
    torch.cuda.synchronize()
    bits = logits.view(torch.int16).numpy().view(np.uint16) if dt == "bf16" else logits.numpy()
    rw, ri = oracle.moe_topk_gating(bits, k, dtype=dt)
    np.testing.assert_array_equal(i.cpu().numpy(), ri)
    np.testing.assert_array_equal(_u16(w), np.asarray(rw).view(np.uint16))
    tw, ti = impl_torch.run(logits, M, E, k)   # the harness reference agrees too
    np.testing.assert_array_equal(ti.numpy(), ri)


@pytest.mark.parametrize("E", [5, 16, 100, 120, 128, 1024])
@pytest.mark.parametrize("k", [1, 2])
@pytest.mark.parametrize("dt", ["fp16", "bf16"])
def test_gating_top2_half_paths(gpu, E, k, dt):
    """k <= 2 on half logits (the 32-bit selection): lanes with whole 16-byte
    chunks (E = 128, 1024), lanes reading element by element (E = 5, 100, 120:
    rows not a 16-byte multiple or a lane's chunk past the row's end), one lane
    per row (E <= 16) and 64 (E = 1024); heavy ties, signed zeros, +-inf, all-
    equal rows, and NaN rows that send their wavefront to the general path.
    Indices exact; weights NaN where the oracle's are and otherwise within one
    unit of the half's last place (the device expf and numpy's may differ by an
    fp32 ulp, which the rounding to a half can carry, as in the filter test)."""
    from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_hip

    _say("gating top2 half", E, k, dt)
    tdt = torch.float16 if dt == "fp16" else torch.bfloat16
    rng = np.random.default_rng(E * 10 + k)
    x = rng.integers(-4, 5, size=(700, E)).astype(np.float32) * 0.5    # heavy ties
    x[:300] = rng.standard_normal((300, E)).astype(np.float32)
    x[310, :] = 0.0
    x[310, E // 2] = -0.0
    x[311, :] = -0.0
    x[312, :] = -np.inf
    x[313, E - 1] = np.inf
    x[314, 0] = np.inf
    x[314, E // 2] = np.inf
    x[315, :] = 1.5
    x[330, E // 3] = np.nan                   # general path for its wavefront (the inf rows stay out of it)
    x[650, 0] = np.nan
    x[651, :] = np.nan
    logits = torch.from_numpy(x).to(tdt)
    w, i = impl_hip.run(logits.to(gpu), logits.shape[0], E, k)
    torch.cuda.synchronize()
    bits = logits.view(torch.int16).numpy().view(np.uint16) if dt == "bf16" else logits.numpy()
    rw, ri = oracle.moe_topk_gating(bits, k, dtype=dt)
    np.testing.assert_array_equal(i.cpu().numpy(), ri)
    got = _u16(w)
    want = np.asarray(rw).view(np.uint16)
    nan_got = np.isnan(w.float().cpu().numpy())
    nan_want = np.isnan(oracle.bf16_bits_to_f32(rw) if dt == "bf16" else rw.astype(np.float32))
    np.testing.assert_array_equal(nan_got, nan_want)
    assert np.abs(got[~nan_got].astype(np.int32) - want[~nan_want].astype(np.int32)).max() <= 1
    # Bit for bit against the general path: the same logits in fp32 take it
    # (k <= 2 in fp32 has no 32-bit shortcut), and its fp32 weights rounded
    # once to the half dtype are what the half path stores.
    w32, i32 = impl_hip.run(logits.float().to(gpu), logits.shape[0], E, k)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(i.cpu().numpy(), i32.cpu().numpy())
    np.testing.assert_array_equal(got[~nan_got], _u16(w32.to(tdt))[~nan_got])


@pytest.mark.parametrize("M", [1024, 20480])
@pytest.mark.parametrize("dt", ["fp16", "bf16", "fp32"])
def test_gating_reference_grid(gpu, M, dt):
    """The reference operator's own case grid (moe_topk_gating/config.yaml: E = 128,
    k = 2, M = 1024..20480, fp16/bf16/fp32, distinct-value "grid" logits): indices
    bit-exact, weights bit-exact in the half dtypes and within 1e-5 in fp32."""
    from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_hip

    _say("gating reference grid", M, dt)
    tdt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[dt]
    logits, M, E, k = T.generate_moe_topk_gating_inputs(M, 128, 2, dtype=tdt, dist="grid", seed=M, device="cpu")
    w, i = impl_hip.run(logits.to(gpu), M, E, k)
    torch.cuda.synchronize()
    bits = logits.view(torch.int16).numpy().view(np.uint16) if dt == "bf16" else logits.numpy()
    rw, ri = oracle.moe_topk_gating(bits, k, dtype=dt)
    np.testing.assert_array_equal(i.cpu().numpy(), ri)
    if dt == "fp32":
        np.testing.assert_allclose(w.cpu().numpy(), rw, atol=1e-5, rtol=1e-5)
    else:
        np.testing.assert_array_equal(_u16(w), np.asarray(rw).view(np.uint16))


# ----------------------------------------------------------------------------- fp8 quant

@pytest.mark.parametrize("M,K", [(8192, 8192), (64, 1024), (3, 24), (17, 2048 * 3), (5, 40000), (256, 16384)])
def test_fp8_quant_matches_oracle(gpu, M, K):
    from tilebench_amd.benchmarks.operators.fp8_act_quant import impl_hip

    _say("fp8_act_quant", M, K)
    (A,) = T.generate_fp8_act_quant_inputs(M, K, seed=M + K, device="cpu")
    q, sa = impl_hip.run(A.to(gpu))
    torch.cuda.synchronize()
    rq, rsa = oracle.fp8_act_quant(A.numpy())
    np.testing.assert_array_equal(sa.cpu().numpy().view(np.uint32), rsa.view(np.uint32))
    got = q.cpu().view(torch.uint8).numpy()
    bad = np.argwhere(got != rq)
    assert bad.size == 0, f"{len(bad)} codes differ, first {bad[:3].tolist()}"


def test_fp8_quant_special_rows(gpu):
    """Zero row, a row whose max maps to exactly 448, subnormal fp16 inputs, +-65504, signed zeros,
    rows holding inf and NaN (the IEEE quotients of the CPU reference)."""
    from tilebench_amd.benchmarks.operators.fp8_act_quant import impl_hip

    _say("fp8_act_quant special rows")
    K = 4096
    rng = np.random.default_rng(5)
    A = rng.standard_normal((8, K)).astype(np.float16)
    A[0] = 0
    A[1, 17] = 448.0
    A[2] = (np.arange(K) % 1024).astype(np.uint16).view(np.float16)        # subnormals and small normals
    A[3, ::2] = np.float16(65504.0)
    A[3, 1::2] = np.float16(-65504.0)
    A[4] = -0.0
    A[4, 9] = 1.0
    A[5] = np.arange(K, dtype=np.uint16).view(np.float16)                    # every bit pattern below 0x1000
    A[6] = (np.arange(K, dtype=np.uint32) * 15 + 0x3C00).astype(np.uint16).view(np.float16)
    A[6][~np.isfinite(A[6])] = 1.0
    A[7, 3] = np.inf                                                        # row max inf: +-0 codes, inf -> NaN
    A[7, 4] = -np.inf
    A = np.concatenate([A, rng.standard_normal((2, K)).astype(np.float16)])
    A[8, 11] = np.nan                                                       # a NaN row: NaN codes
    A[9, 12] = np.uint16(0xFE00).view(np.float16)                           # a NaN with the sign bit set
    A[9, 13] = -np.inf
    q, sa = impl_hip.run(torch.from_numpy(A).to(gpu))
    torch.cuda.synchronize()
    rq, rsa = oracle.fp8_act_quant(A)
    np.testing.assert_array_equal(sa.cpu().numpy().view(np.uint32), rsa.view(np.uint32))
    np.testing.assert_array_equal(q.cpu().view(torch.uint8).numpy(), rq)


# ----------------------------------------------------------------------------- W4A16 GEMM

def _w4a16_check(gpu, M, K, N, G, seed):
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip

    _say("w4a16_gemm", M, K, N, G)
    A, p, s, z, G = T.generate_w4a16_gemm_inputs(M, K, N, G, seed=seed, device="cpu")
    Y = impl_hip.run(A.to(gpu), p.to(gpu), s.to(gpu), z.to(gpu), G)
    torch.cuda.synchronize()
    ref = oracle.w4a16_gemm(A.numpy(), p.numpy(), s.numpy(), z.numpy(), G)
    got = Y.cpu().numpy()
    np.testing.assert_allclose(got.astype(np.float32), ref.astype(np.float32), atol=1e-2, rtol=1e-2)
    return got, ref


@pytest.mark.parametrize("M,K,N,G", [(1, 4096, 11008, 128), (16, 4096, 11008, 128), (256, 512, 512, 128),
                                     (300, 256, 264, 64), (7, 1024, 1000, 128), (16, 64, 8, 64), (1, 128, 2048, 128),
                                     (512, 4096, 1024, 128), (33, 384, 392, 128), (5, 2048, 1032, 64)])
def test_w4a16_gemm_matches_oracle(gpu, M, K, N, G):
    _w4a16_check(gpu, M, K, N, G, seed=M + N)


@pytest.mark.parametrize("M,K,N,G", [(257, 64, 520, 64), (257, 128, 520, 64), (257, 192, 520, 64),
                                     (257, 320, 520, 64), (3000, 192, 11008, 64)])
def test_w4a16_prefill_short_k(gpu, M, K, N, G):
    """Prefill K loops of 1, 2, 3 and 5 steps: a step's loads go out in four
    parts spread over two steps, the prologue issues only the first part of the
    third stage, and every load past the last step reads nothing.  M = 3000 x
    N = 11008 also runs the 192-row tiles (its last tile columns)."""
    _w4a16_check(gpu, M, K, N, G, seed=M + K)


def test_w4a16_gemm_full_prefill(gpu):
    """BASELINE config 1 at M = 4096: checked against the oracle on a row sample
    (the full fp32 CPU product takes minutes) and for finiteness everywhere."""
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip

    M, K, N, G = 4096, 4096, 11008, 128
    _say("w4a16_gemm full prefill", M, K, N, G)
    A, p, s, z, G = T.generate_w4a16_gemm_inputs(M, K, N, G, seed=1, device="cpu")
    Y = impl_hip.run(A.to(gpu), p.to(gpu), s.to(gpu), z.to(gpu), G)
    torch.cuda.synchronize()
    Yc = Y.cpu().numpy()
    assert np.isfinite(Yc.astype(np.float32)).all()
    rows = np.random.default_rng(0).choice(M, 96, replace=False)
    ref = oracle.w4a16_gemm(A.numpy()[rows], p.numpy(), s.numpy(), z.numpy(), G)
    np.testing.assert_allclose(Yc[rows].astype(np.float32), ref.astype(np.float32), atol=1e-2, rtol=1e-2)


def test_w4a16_prefill_192_row_tail(gpu):
    """M = 3000, N = 11008: 12 x 43 = 516 tiles of 256 x 256 would leave a third
    round of 4 tiles on 256 CUs, so the launch covers tile columns 10 .. 42 with
    16 tiles of 192 rows each instead (the last row of tiles ragged: rows
    2880 .. 2999).  Rows from every part, the ragged rows included, against the
    oracle."""
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip

    M, K, N, G = 3000, 512, 11008, 128
    _say("w4a16_gemm prefill with 192-row tail tiles", M, K, N, G)
    A, p, s, z, G = T.generate_w4a16_gemm_inputs(M, K, N, G, seed=5, device="cpu")
    Y = impl_hip.run(A.to(gpu), p.to(gpu), s.to(gpu), z.to(gpu), G)
    torch.cuda.synchronize()
    Yc = Y.cpu().numpy()
    rows = np.concatenate([np.random.default_rng(1).choice(2880, 64, replace=False), np.arange(2880, 3000)])
    ref = oracle.w4a16_gemm(A.numpy()[rows], p.numpy(), s.numpy(), z.numpy(), G)
    np.testing.assert_allclose(Yc[rows].astype(np.float32), ref.astype(np.float32), atol=1e-2, rtol=1e-2)


def test_w4a16_decode_repeat_calls_reuse_workspace(gpu):
    """The split-K counters must be back at zero after each call: three calls in a row agree."""
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip

    _say("w4a16_gemm decode repeat")
    A, p, s, z, G = T.generate_w4a16_gemm_inputs(16, 4096, 11008, 128, seed=5, device="cpu")
    args = (A.to(gpu), p.to(gpu), s.to(gpu), z.to(gpu), G)
    outs = [impl_hip.run(*args) for _ in range(3)]
    torch.cuda.synchronize()
    first = outs[0].cpu()
    for i, o in enumerate(outs[1:], 1):
        diff = (o.cpu().view(torch.int16) != first.view(torch.int16)).nonzero()
        assert diff.numel() == 0, (f"call {i}: {diff.shape[0]} outputs differ from call 0, first "
                                   f"{diff[:4].tolist()}: {[float(o[m, n]) for m, n in diff[:4].tolist()]} vs "
                                   f"{[float(first[m, n]) for m, n in diff[:4].tolist()]}")


@pytest.mark.parametrize("M", [16, 3])
def test_w4a16_decode_alternating_inputs(gpu, M):
    """Back-to-back decode calls on two different inputs of one shape: every
    result matches its own oracle (stale split-K partials would mix them)."""
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip

    _say("w4a16_gemm decode alternating", M)
    K, N, G = 2048, 4096, 128
    sets = [T.generate_w4a16_gemm_inputs(M, K, N, G, seed=s, device="cpu") for s in (21, 22)]
    refs = [oracle.w4a16_gemm(A.numpy(), p.numpy(), s.numpy(), z.numpy(), G) for A, p, s, z, G in sets]
    dev = [tuple(t.to(gpu) if isinstance(t, torch.Tensor) else t for t in x) for x in sets]
    outs = [impl_hip.run(*dev[i % 2]) for i in range(6)]
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        np.testing.assert_allclose(o.cpu().numpy().astype(np.float32), refs[i % 2].astype(np.float32),
                                   atol=1e-2, rtol=1e-2, err_msg=f"call {i}")
    for i in range(2, 6):
        assert torch.equal(outs[i], outs[i % 2]), f"call {i} differs from call {i % 2}"


def test_w4a16_decode_graph_survives_workspace_growth(gpu):
    """A graph captured at M = 1 keeps the workspace address it was captured
    with; a later eager M = 16 call needs a larger workspace.  The old buffer
    must stay alive and zeroed, so every replay (with eager calls between the
    replays) still matches the oracle."""
    from tilebench_amd import runtime as rt
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip

    _say("w4a16_gemm decode graph + workspace growth")
    key = str(gpu)
    if key in rt._workspaces:  # start from no cached workspace; the old one stays alive
        rt._retired.append(rt._workspaces.pop(key))
    K, N, G = 4096, 11008, 128
    small = T.generate_w4a16_gemm_inputs(1, K, N, G, seed=31, device="cpu")
    big = T.generate_w4a16_gemm_inputs(16, K, N, G, seed=32, device="cpu")
    refs = [oracle.w4a16_gemm(A.numpy(), p.numpy(), s.numpy(), z.numpy(), G) for A, p, s, z, G in (small, big)]
    d_small = tuple(t.to(gpu) if isinstance(t, torch.Tensor) else t for t in small)
    d_big = tuple(t.to(gpu) if isinstance(t, torch.Tensor) else t for t in big)
    impl_hip.run(*d_small)  # allocates the (small) workspace eagerly
    torch.cuda.synchronize()
    ws_small = rt._workspaces[key].data_ptr()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_graph = impl_hip.run(*d_small)
    y_big = impl_hip.run(*d_big)  # grows the workspace: a new buffer becomes the cached one
    torch.cuda.synchronize()
    assert rt._workspaces[key].data_ptr() != ws_small, "M = 16 should have needed a larger workspace"
    assert any(b.data_ptr() == ws_small for b in rt._retired), "the captured workspace was released"
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_allclose(y_graph.cpu().numpy().astype(np.float32), refs[0].astype(np.float32),
                                   atol=1e-2, rtol=1e-2, err_msg=f"replay {i}")
        y_big = impl_hip.run(*d_big)
        torch.cuda.synchronize()
        np.testing.assert_allclose(y_big.cpu().numpy().astype(np.float32), refs[1].astype(np.float32),
                                   atol=1e-2, rtol=1e-2, err_msg=f"eager call after replay {i}")
    del graph


def _slab_layout(packed: np.ndarray) -> np.ndarray:
    """The slab layout of packed int4 weights [K, N/2] as include/tbhip.h
    defines it for tb_w4a16_repack_slabs, restated with numpy fancy indexing:
    slab s, unit u, lane l, word b holds the codes of column 64 s + 16 b + l % 16
    at rows 32 u + 8 (l / 16) + i, code i at bit (i % 2) * 16 + (i / 2) * 4."""
    K, half = packed.shape
    N = 2 * half
    q = np.empty((K, N), np.uint32)
    q[:, 0::2] = packed & 15
    q[:, 1::2] = packed >> 4
    s = np.arange(N // 64)[:, None, None, None]
    u = np.arange(K // 32)[None, :, None, None]
    l = np.arange(64)[None, None, :, None]
    b = np.arange(4)[None, None, None, :]
    words = np.zeros((N // 64, K // 32, 64, 4), np.uint32)
    for i in range(8):
        words |= q[32 * u + 8 * (l // 16) + i, 64 * s + 16 * b + l % 16] << np.uint32((i % 2) * 16 + (i // 2) * 4)
    return words.reshape(-1).view(np.uint8)


@pytest.mark.parametrize("K,N", [(4096, 11008), (256, 128)])
def test_w4a16_slab_layout_on_the_gpu(gpu, K, N):
    """formats.w4a16_to_slabs on a GPU tensor (tb_w4a16_repack_slabs) equals the
    layout restated on the host, byte for byte, and maps back exactly."""
    _say("w4a16 slab layout", K, N)
    _, p, _, _, _ = T.generate_w4a16_gemm_inputs(1, K, N, 128, seed=K + N, device="cpu")
    wr = formats.w4a16_to_slabs(p.to(gpu))
    torch.cuda.synchronize()
    assert tuple(wr.shape) == formats.slab_shape(K, N)
    np.testing.assert_array_equal(wr.cpu().numpy().reshape(-1), _slab_layout(p.numpy()))
    assert torch.equal(formats.w4a16_from_slabs(wr).cpu(), p)


# every slab_decode<UPW, UPG> instance: UPW = K / 512, UPG = G / 32
@pytest.mark.parametrize("M,K,N,G", [(1, 4096, 11008, 128), (16, 4096, 11008, 128), (5, 4096, 11008, 128),
                                     (4, 4096, 1024, 64), (9, 2048, 768, 64), (3, 2048, 512, 128),
                                     (16, 1024, 256, 64), (2, 1024, 64, 64)])
def test_w4a16_slab_decode_matches_oracle(gpu, M, K, N, G):
    """The slab decode (weights in the slab layout) against the oracle, three
    calls in a row bit-identical, and the split-K decode over the packed layout
    close to it."""
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip

    _say("w4a16 slab decode", M, K, N, G)
    assert impl_hip.slab_shape_ok(M, N, K, G)
    A, p, s, z, G = T.generate_w4a16_gemm_inputs(M, K, N, G, seed=7 * M + K, device="cpu")
    rows = (A.to(gpu), p.to(gpu), s.to(gpu), z.to(gpu), G)
    slabs = (rows[0], formats.w4a16_to_slabs(rows[1]), rows[2], rows[3], G)
    outs = [impl_hip.run(*slabs) for _ in range(3)]
    assert impl_hip.get_last_config()["kernel"] == "w4a16_slab_decode"
    split = impl_hip.run(*rows)
    assert impl_hip.get_last_config()["kernel"] == "w4a16_decode"
    torch.cuda.synchronize()
    ref = oracle.w4a16_gemm(A.numpy(), p.numpy(), s.numpy(), z.numpy(), G)
    np.testing.assert_allclose(outs[0].cpu().numpy().astype(np.float32), ref.astype(np.float32), atol=1e-2, rtol=1e-2)
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    np.testing.assert_allclose(split.float().cpu().numpy(), outs[0].float().cpu().numpy(), atol=1e-2, rtol=1e-2)


def test_w4a16_slab_layout_refuses_prefill_shapes(gpu):
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip

    A, p, s, z, G = T.generate_w4a16_gemm_inputs(17, 1024, 256, 64, seed=3, device="cpu")
    with pytest.raises(ValueError, match="decode format"):
        impl_hip.run(A.to(gpu), formats.w4a16_to_slabs(p.to(gpu)), s.to(gpu), z.to(gpu), G)


@pytest.mark.parametrize("layout", ["rows", "slabs"])
@pytest.mark.parametrize("M", [1, 16, 64])
def test_w4a16_in_place_weight_update_is_seen(gpu, layout, M):
    """Weights, scales and zero-points rewritten in place (same tensors, same
    addresses) between two calls: the second call multiplies by the new
    values.  run() keeps nothing between calls, so no layout can return a
    product of the old weights."""
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip

    if layout == "slabs" and M > 16:
        pytest.skip("the slab layout is a decode format")
    K, N, G = 4096, 11008, 128
    _say("w4a16 in-place weight update", layout, M)
    old = T.generate_w4a16_gemm_inputs(M, K, N, G, seed=51, device="cpu")
    new = T.generate_w4a16_gemm_inputs(M, K, N, G, seed=52, device="cpu")

    def dev(x):
        A, p, s, z, g = x
        p = p.to(gpu)
        return [A.to(gpu), formats.w4a16_to_slabs(p) if layout == "slabs" else p, s.to(gpu), z.to(gpu), g]

    d_old, d_new = dev(old), dev(new)
    y_old = impl_hip.run(*d_old)
    ptrs = [t.data_ptr() for t in d_old[1:4]]
    for dst, src in zip(d_old[1:4], d_new[1:4]):
        dst.copy_(src)
    assert [t.data_ptr() for t in d_old[1:4]] == ptrs
    y_new = impl_hip.run(*d_old)
    torch.cuda.synchronize()
    A = old[0].numpy()
    for y, (_, p, s, z, _g), what in ((y_old, old, "before"), (y_new, new, "after")):
        ref = oracle.w4a16_gemm(A, p.numpy(), s.numpy(), z.numpy(), G)
        np.testing.assert_allclose(y.cpu().numpy().astype(np.float32), ref.astype(np.float32), atol=1e-2, rtol=1e-2,
                                   err_msg=f"{what} the in-place update")


def test_w4a16_slab_decode_in_a_graph_sees_weight_updates(gpu):
    """A graph captured on slab-layout weights replays the slab decode; the
    weights rewritten in place between replays (eager work and a sync between
    them) give the new product on the next replay."""
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip

    _say("w4a16 slab decode in a graph")
    K, N, G = 4096, 11008, 128
    sets = [T.generate_w4a16_gemm_inputs(1, K, N, G, seed=s, device="cpu") for s in (41, 42)]
    A = sets[0][0]
    refs = [oracle.w4a16_gemm(A.numpy(), p.numpy(), s.numpy(), z.numpy(), G) for _, p, s, z, _g in sets]
    slabs = [formats.w4a16_to_slabs(x[1].to(gpu)) for x in sets]
    d = (A.to(gpu), slabs[0].clone(), sets[0][2].to(gpu), sets[0][3].to(gpu), G)
    scales = [x[2].to(gpu) for x in sets]
    zeros = [x[3].to(gpu) for x in sets]
    impl_hip.run(*d)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = impl_hip.run(*d)
    assert impl_hip.get_last_config()["kernel"] == "w4a16_slab_decode"
    for i in range(4):
        j = i % 2
        d[1].copy_(slabs[j])
        d[2].copy_(scales[j])
        d[3].copy_(zeros[j])
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_allclose(y.cpu().numpy().astype(np.float32), refs[j].astype(np.float32), atol=1e-2,
                                   rtol=1e-2, err_msg=f"replay {i}")
        impl_hip.run(*d)   # eager work between the replays
        torch.cuda.synchronize()
    del g


# ----------------------------------------------------------------------------- fp8 GEMM

def _fp8_gemm_check(gpu, M, N, K, seed):
    from tilebench_amd.benchmarks.operators.fp8_scaled_gemm import impl_hip

    _say("fp8_scaled_gemm", M, N, K)
    Aq, Wq, sa, sw = T.generate_fp8_scaled_gemm_inputs(M, N, K, seed=seed, device="cpu")
    Y = impl_hip.run(Aq.to(gpu), Wq.to(gpu), sa.to(gpu), sw.to(gpu))
    torch.cuda.synchronize()
    ref = oracle.bf16_bits_to_f32(oracle.fp8_scaled_gemm(Aq.view(torch.uint8).numpy(),
                                                         Wq.contiguous().view(torch.uint8).numpy(),
                                                         sa.numpy(), sw.numpy()))
    got = Y.float().cpu().numpy()
    np.testing.assert_allclose(got, ref, atol=1e-2, rtol=1e-2)
    return got, ref


@pytest.mark.parametrize("M,N,K", [(256, 256, 128), (512, 768, 1024), (300, 200, 256), (64, 8, 128),
                                   (1024, 1024, 2048)])
def test_fp8_gemm_matches_oracle(gpu, M, N, K):
    _fp8_gemm_check(gpu, M, N, K, seed=M + N + K)


def test_fp8_gemm_full_size_rows(gpu):
    """BASELINE config 2 (8192^3): rows sampled against the oracle, all finite."""
    from tilebench_amd.benchmarks.operators.fp8_scaled_gemm import impl_hip

    M = N = K = 8192
    _say("fp8_scaled_gemm full", M, N, K)
    Aq, Wq, sa, sw = T.generate_fp8_scaled_gemm_inputs(M, N, K, seed=2, device="cpu")
    Y = impl_hip.run(Aq.to(gpu), Wq.to(gpu), sa.to(gpu), sw.to(gpu)).float().cpu().numpy()
    assert np.isfinite(Y).all()
    rows = np.random.default_rng(1).choice(M, 48, replace=False)
    ref = oracle.bf16_bits_to_f32(oracle.fp8_scaled_gemm(Aq.view(torch.uint8).numpy()[rows],
                                                         Wq.contiguous().view(torch.uint8).numpy(),
                                                         sa.numpy()[rows], sw.numpy()))
    np.testing.assert_allclose(Y[rows], ref, atol=1e-2, rtol=1e-2)


def test_fp8_gemm_rounding_ties_and_specials(gpu):
    """The epilogue's bf16 rounding and special values, on exact sums.

    Sums of 1 and e4m3 subnormals land exactly on bf16 rounding ties (1 + 2^-8
    rounds to 1, 1 + 3 * 2^-8 to 1 + 2^-6: to even) and next to them (1 + 5 *
    2^-9 rounds up), in both signs; an e4m3 NaN code poisons its row; an
    infinite column scale gives +-inf, or NaN where the sum is zero.  With unit
    scales the oracle's value is exact, so finite outputs must match it bit for
    bit and NaNs position for position."""
    from tilebench_amd.benchmarks.operators.fp8_scaled_gemm import impl_hip

    M, N, K = 64, 64, 128
    _say("fp8_scaled_gemm specials", M, N, K)
    A = np.zeros((M, K), np.uint8)
    W = np.zeros((K, N), np.uint8)
    A[0, 0] = A[0, 1] = 0x38            # +1, +1
    A[1, 0] = A[1, 1] = 0xB8            # -1, -1
    A[2, 0], A[2, 1] = 0x7F, 0x38       # NaN poisons row 2
    A[4, 0] = 0x38                      # row 4: exactly 1 (+ W[1, n] * 0)
    W[0, :] = 0x38                      # 1.0 in every column
    W[1, 0], W[1, 1], W[1, 2] = 0x02, 0x06, 0x05  # 2^-8, 3 * 2^-8, 5 * 2^-9
    sa = np.ones(M, np.float32)
    sw = np.ones(N, np.float32)
    sw[5] = np.inf
    to_t = lambda x: torch.from_numpy(x).view(torch.float8_e4m3fn)
    Y = impl_hip.run(to_t(A).to(gpu), to_t(W).to(gpu), torch.from_numpy(sa).to(gpu), torch.from_numpy(sw).to(gpu))
    torch.cuda.synchronize()
    got = Y.view(torch.int16).cpu().numpy().view(np.uint16)
    with np.errstate(invalid="ignore"):  # 0 * inf in column 5 is the NaN being tested
        ref = oracle.fp8_scaled_gemm(A, W, sa, sw)
    gotf, reff = oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref)
    assert np.array_equal(np.isnan(gotf), np.isnan(reff))
    fin = ~np.isnan(reff)
    assert np.array_equal(got[fin], ref[fin])
    assert got[0, 0] == 0x3F80 and got[0, 1] == 0x3F82 and got[0, 2] == 0x3F81
    assert got[1, 0] == 0xBF80 and got[1, 1] == 0xBF82 and got[1, 2] == 0xBF81
    assert np.isnan(gotf[2]).all() and np.isnan(gotf[3, 5]) and gotf[0, 5] == np.inf and gotf[1, 5] == -np.inf


def test_host_tensors_are_refused(gpu):
    """A host tensor among the inputs raises ValueError before any launch (its
    address would otherwise reach a kernel as a device address)."""
    from tilebench_amd.benchmarks.operators.fp8_scaled_gemm import impl_hip as f8
    from tilebench_amd.benchmarks.operators.int4_dequant import impl_hip as dq
    from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_hip as gt
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip as wg

    _say("host tensors refused")
    p, s, z, K, N, G = T.generate_int4_dequant_inputs(256, 64, 128, seed=1, device="cpu")
    with pytest.raises(ValueError, match="is on cpu"):
        dq.run(p.to(gpu), s, z.to(gpu), K, N, G)
    A, wp, ws, wz, G = T.generate_w4a16_gemm_inputs(32, 256, 64, 128, seed=2, device="cpu")
    with pytest.raises(ValueError, match="input 0 is on cpu"):
        wg.run(A, wp.to(gpu), ws.to(gpu), wz.to(gpu), G)
    logits, M, E, k = T.generate_moe_topk_gating_inputs(64, 64, 8, seed=3, device="cpu")
    with pytest.raises(ValueError, match="is on cpu"):
        gt.run(logits, M, E, k)
    Aq, Wq, sa, sw = T.generate_fp8_scaled_gemm_inputs(256, 256, 128, seed=4, device="cpu")
    with pytest.raises(ValueError, match="input 3 is on cpu"):
        f8.run(Aq.to(gpu), Wq.to(gpu), sa.to(gpu), sw)
    torch.cuda.synchronize()


def test_golden_fixtures_on_gpu(gpu):
    """Every committed golden fixture reproduced by the GPU kernels."""
    import os
    from tilebench_amd.benchmarks.operators.int4_dequant import impl_hip as dq
    from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_hip as gt
    from tilebench_amd.benchmarks.operators.fp8_act_quant import impl_hip as fq
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip as wg
    from tilebench_amd.benchmarks.operators.fp8_scaled_gemm import impl_hip as fg

    _say("golden fixtures")
    gd = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    ld = lambda n: dict(np.load(os.path.join(gd, n + ".npz")))
    d = lambda a: torch.from_numpy(a).to(gpu)
    f = ld("int4_dequant")
    K, N = f["out"].shape
    out = dq.run(d(f["packed"]), d(f["scales"]), d(f["zeros"]), K, N, int(f["group"]))
    np.testing.assert_array_equal(_u16(out), f["out"].view(np.uint16))
    f = ld("moe_topk_gating")
    w, i = gt.run(d(f["logits"]), *f["logits"].shape, int(f["k"]))
    np.testing.assert_array_equal(i.cpu().numpy(), f["indices"])
    np.testing.assert_allclose(w.cpu().numpy(), f["weights"], atol=1e-5, rtol=1e-5)
    f = ld("fp8_act_quant")
    q, sa = fq.run(d(f["A"]))
    np.testing.assert_array_equal(q.cpu().view(torch.uint8).numpy(), f["codes"])
    f = ld("w4a16_gemm")
    Y = wg.run(d(f["A"]), d(f["packed"]), d(f["scales"]), d(f["zeros"]), int(f["group"]))
    np.testing.assert_allclose(Y.cpu().numpy().astype(np.float32), f["Y"].astype(np.float32), atol=1e-2, rtol=1e-2)
    f = ld("fp8_scaled_gemm")
    aq = d(f["Aq"]).view(torch.float8_e4m3fn)
    wq = d(np.ascontiguousarray(f["Wq"].T)).view(torch.float8_e4m3fn).t()
    Y = fg.run(aq, wq, d(f["sa"]), d(f["sw"]))
    np.testing.assert_allclose(Y.float().cpu().numpy(), oracle.bf16_bits_to_f32(f["Y"]), atol=1e-2, rtol=1e-2)


# ----------------------------------------------------------------------------- grouped MoE W4A16

@pytest.mark.parametrize("tokens,topk,E,K,N,pad", [(512, 2, 8, 256, 1408, 128), (300, 4, 16, 512, 264, 16),
                                                    (64, 1, 4, 128, 64, 64), (1000, 8, 64, 256, 512, 128),
                                                    (400, 2, 8, 384, 1408, 128)])
def test_grouped_gemm_matches_oracle(gpu, tokens, topk, E, K, N, pad):
    from tilebench_amd.benchmarks.operators.moe_w4a16_grouped_gemm import impl_hip

    _say("moe_w4a16_grouped_gemm", tokens, topk, E, K, N, pad)
    A, p, s, z, off, G = T.generate_moe_w4a16_grouped_gemm_inputs(tokens, topk, E, K, N, 128, pad=pad,
                                                                  seed=tokens + E, device="cpu")
    Y = impl_hip.run(A.to(gpu), p.to(gpu), s.to(gpu), z.to(gpu), off.to(gpu), G)
    torch.cuda.synchronize()
    ref = oracle.moe_w4a16_grouped_gemm(A.numpy(), p.numpy(), s.numpy(), z.numpy(), off.numpy(), G)
    np.testing.assert_allclose(Y.cpu().numpy().astype(np.float32), ref.astype(np.float32), atol=1e-2, rtol=1e-2)


def test_grouped_gemm_segments_equal_dense_kernel(gpu):
    """Each expert's rows of the grouped product equal the dense W4A16 kernel on
    that expert (bit for bit: same tile code, same summation order)."""
    from tilebench_amd.benchmarks.operators.moe_w4a16_grouped_gemm import impl_hip as gg
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip as wg

    _say("grouped vs dense")
    A, p, s, z, off, G = T.generate_moe_w4a16_grouped_gemm_inputs(2048, 8, 16, 1024, 1408, 128, pad=128,
                                                                  seed=9, device="cpu")
    Ad, pd, sd, zd = A.to(gpu), p.to(gpu), s.to(gpu), z.to(gpu)
    Y = gg.run(Ad, pd, sd, zd, off.to(gpu), G)
    o = off.tolist()
    last = {(o[e + 1] - o[e]) % 256 for e in range(16) if o[e + 1] - o[e] > 16}
    # both last-tile shapes run: 256 rows (remainder 0) and 128 rows (remainder 128)
    assert {0, 128} <= last, last
    for e in range(16):
        lo, hi = o[e], o[e + 1]
        if hi - lo > 16:
            Ye = wg.run(Ad[lo:hi], pd[e], sd[e], zd[e], G)
            assert torch.equal(Y[lo:hi], Ye), f"expert {e}"


def test_grouped_gemm_full_config_rows(gpu):
    """BASELINE config 4 (64 experts, 16384 tokens x top-8, Zipf 1.1): rows of the
    heaviest and lightest experts checked against the oracle."""
    from tilebench_amd.benchmarks.operators.moe_w4a16_grouped_gemm import impl_hip

    _say("grouped full config 4")
    A, p, s, z, off, G = T.generate_moe_w4a16_grouped_gemm_inputs(16384, 8, 64, 4096, 1408, 128, seed=4,
                                                                  device="cpu")
    Y = impl_hip.run(A.to(gpu), p.to(gpu), s.to(gpu), z.to(gpu), off.to(gpu), G).cpu().numpy()
    o = off.numpy()
    sizes = np.diff(o)
    for e in (int(np.argmax(sizes)), int(np.argmin(np.where(sizes > 0, sizes, 1 << 30)))):
        lo = o[e]
        rows = slice(lo, min(lo + 64, o[e + 1]))
        ref = oracle.w4a16_gemm(A.numpy()[rows], p.numpy()[e], s.numpy()[e], z.numpy()[e], G)
        np.testing.assert_allclose(Y[rows].astype(np.float32), ref.astype(np.float32), atol=1e-2, rtol=1e-2)
    assert np.isfinite(Y.astype(np.float32)).all()


# ----------------------------------------------------------------------------- reference analog operators

@pytest.mark.parametrize("M,N,tile_size,dt", [(512, 512, 128, "fp16"), (1000, 1000, 128, "bf16"),
                                               (2048, 2048, 128, "fp32"), (37, 45, 7, "fp16"), (64, 96, 16, "bf16"),
                                               (10240, 10240, 128, "fp16")])
def test_weight_dequant_matches_oracle(gpu, M, N, tile_size, dt):
    from tilebench_amd.benchmarks.operators.weight_dequant import impl_hip

    _say("weight_dequant", M, N, tile_size, dt)
    tdt = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}[dt]
    X, S, M, N, tile = T.generate_weight_dequant_inputs(M, tile_size, dtype=tdt, N=N, seed=M, device="cpu")
    Y = impl_hip.run(X.to(gpu), S.to(gpu), M, N, tile)
    torch.cuda.synchronize()
    if dt == "bf16":
        ref = oracle.weight_dequant(X.view(torch.int16).numpy().view(np.uint16),
                                    S.view(torch.int16).numpy().view(np.uint16), tile, dt)
        np.testing.assert_array_equal(_u16(Y), ref)
    else:
        ref = oracle.weight_dequant(X.numpy(), S.numpy(), tile, dt)
        got = Y.cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint32 if dt == "fp32" else np.uint16),
                                      ref.view(np.uint32 if dt == "fp32" else np.uint16))


@pytest.mark.parametrize("rows,cols", [(512, 512), (4096, 8192), (33, 100), (7, 16),
                                       (3, 6160), (65543, 32)])   # a chunk ending in its second half; > 65535 rows
def test_dequantize_rowwise_matches_oracle(gpu, rows, cols):
    from tilebench_amd.benchmarks.operators.dequantize_rowwise import impl_hip

    _say("dequantize_rowwise", rows, cols)
    x, s = T.generate_dequantize_rowwise_inputs(rows, cols, seed=rows + cols, device="cpu")
    y = impl_hip.run(x.to(gpu), s.to(gpu))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u16(y), oracle.dequantize_rowwise(x.numpy(), s.numpy()).view(np.uint16))


@pytest.mark.parametrize("n", [1 << 20, 20 * (1 << 20), 1001, 3])
def test_quantize_global_matches_oracle(gpu, n):
    from tilebench_amd.benchmarks.operators.quantize_global import impl_hip

    _say("quantize_global", n)
    (x,) = T.generate_quantize_global_inputs(n, seed=n % 97, device="cpu")
    x[: min(n, 8)] = torch.tensor([65504.0, 65520.0, -1e-8, 2.0 ** -24, 2.0 ** -25, 3.0 * 2.0 ** -26, 1e30, -0.0])[: min(n, 8)]
    y = impl_hip.run(x.to(gpu))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u16(y), oracle.quantize_global(x.numpy()).view(np.uint16))


# ----------------------------------------------------------------------------- plain GEMM operators

def _rows(M, n, seed):
    return np.sort(np.random.default_rng(seed).choice(M, min(M, n), replace=False))


@pytest.mark.parametrize("M,N,K", [(256, 256, 1024), (100, 264, 512), (2048, 2048, 1024), (2048, 2048, 20480),
                                   (1024, 1024, 128), (4096, 4096, 1024),
                                   # split-K: 4 splits over 37 K steps with ragged tile edges; 8 splits
                                   (600, 520, 4736), (256, 512, 16384)])
def test_matmul_int8_bit_exact(gpu, M, N, K):
    from tilebench_amd.benchmarks.operators.matmul_int8 import impl_hip

    _say("matmul_int8", M, N, K)
    a, b = T.generate_matmul_int8_inputs(M, N, K, seed=M + K, device="cpu")
    out = impl_hip.run(a.to(gpu), b.to(gpu))
    torch.cuda.synchronize()
    rows = _rows(M, 128, K)
    np.testing.assert_array_equal(out.cpu().numpy()[rows], oracle.matmul_int8(a.numpy()[rows], b.numpy()))
    splits = impl_hip.get_last_config()["k_splits"]
    assert splits == {(2048, 2048, 20480): 4, (600, 520, 4736): 4, (256, 512, 16384): 8}.get((M, N, K), 1)


@pytest.mark.parametrize("M,N,K", [(512, 512, 1024), (300, 136, 256), (4096, 4096, 4096), (4096, 4096, 20480)])
def test_matmul_fp16(gpu, M, N, K):
    from tilebench_amd.benchmarks.operators.matmul_fp32_fp16_fp8 import impl_hip

    _say("matmul fp16", M, N, K)
    a, b = T.generate_matmul_fp32_fp16_fp8_inputs(M, N, K, dtype=torch.float16, seed=M + K, device="cpu")
    out = impl_hip.run(a.to(gpu), b.to(gpu))
    torch.cuda.synchronize()
    rows = _rows(M, 128, K)
    ref = oracle.matmul_f16(a.numpy()[rows], b.numpy()).astype(np.float32)
    np.testing.assert_allclose(out.cpu().numpy()[rows].astype(np.float32), ref, atol=2e-3, rtol=2e-3)


@pytest.mark.parametrize("M,N,K", [(512, 512, 1024), (300, 136, 64), (4096, 4096, 2048), (4096, 4096, 20480)])
def test_matmul_fp32_three_bf16_products(gpu, M, N, K):
    """fp32 operands through hi/lo bf16 splits: within 1e-4 of the float64 product,
    an order of magnitude tighter than TF32 (10 mantissa bits) would allow."""
    from tilebench_amd.benchmarks.operators.matmul_fp32_fp16_fp8 import impl_hip

    _say("matmul fp32", M, N, K)
    a, b = T.generate_matmul_fp32_fp16_fp8_inputs(M, N, K, dtype=torch.float32, seed=M + K, device="cpu")
    out = impl_hip.run(a.to(gpu), b.to(gpu))
    torch.cuda.synchronize()
    rows = _rows(M, 128, K)
    ref = oracle.matmul_f32(a.numpy()[rows], b.numpy())
    np.testing.assert_allclose(out.cpu().numpy()[rows], ref, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("M,N,K", [(512, 512, 1024), (300, 136, 128), (4096, 4096, 4096), (4096, 4096, 20480)])
def test_matmul_fp8(gpu, M, N, K):
    """e4m3(bf16(a @ b)): fp32 accumulation against the oracle's float64 may move a
    bf16 rounding on rare values, so codes agree exactly on > 99.5 % and the
    decoded values never differ by more than one e4m3 step."""
    from tilebench_amd.benchmarks.operators.matmul_fp32_fp16_fp8 import impl_hip

    _say("matmul fp8", M, N, K)
    a, b = T.generate_matmul_fp32_fp16_fp8_inputs(M, N, K, dtype=torch.float8_e4m3fn, seed=M + K, device="cpu")
    ag, bg = a.to(gpu), b.to(gpu)
    out = impl_hip.run(ag, bg)
    out2 = impl_hip.run(ag, bg)   # second call: cached transposed operand
    torch.cuda.synchronize()
    rows = _rows(M, 128, K)
    got = out.cpu().view(torch.uint8).numpy()[rows]
    ref = oracle.matmul_fp8(a.view(torch.uint8).numpy()[rows], b.view(torch.uint8).numpy())
    assert (got == ref).mean() > 0.995
    g, r = oracle.e4m3_to_f32(got), oracle.e4m3_to_f32(ref)
    step = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(r), 2.0 ** -6))) - 3)
    assert (np.abs(g - r) <= step + 1e-12).all()
    assert torch.equal(out.view(torch.uint8), out2.view(torch.uint8))
