"""Checkpoint format converters (GPTQ, AWQ, fp8) against independent
restatements of the packers' published conventions (pure-Python bit loops on
small shapes), exact round trips, and torch's own fp8 decoders."""
import numpy as np
import pytest
import torch

import oracle
from tilebench_amd import formats as F


def _i32(u):
    return int(u) - (1 << 32) if u >= 1 << 31 else int(u)


def gptq_pack_loop(q, z, zero_offset=1):
    """AutoGPTQ v1 packing written out bit by bit: qweight word [i, n] holds
    rows 8i..8i+7 of column n (row 8i + j in bits 4j..); qzeros word [g, i]
    holds zero - 1 of columns 8i..8i+7."""
    K, N = q.shape
    qw = np.zeros((K // 8, N), dtype=np.int64)
    for i in range(K // 8):
        for n in range(N):
            word = 0
            for j in range(8):
                word |= int(q[8 * i + j, n]) << (4 * j)
            qw[i, n] = _i32(word)
    ng = z.shape[0]
    qz = np.zeros((ng, N // 8), dtype=np.int64)
    for g in range(ng):
        for i in range(N // 8):
            word = 0
            for j in range(8):
                word |= ((int(z[g, 8 * i + j]) - zero_offset) & 0xF) << (4 * j)
            qz[g, i] = _i32(word)
    return torch.from_numpy(qw.astype(np.int32)), torch.from_numpy(qz.astype(np.int32))


def awq_pack_loop(codes):
    """AutoAWQ GEMM packing: word [r, i] holds columns 8i + (0,2,4,6,1,3,5,7)[j]
    in nibble j."""
    R, N = codes.shape
    order = [0, 2, 4, 6, 1, 3, 5, 7]
    out = np.zeros((R, N // 8), dtype=np.int64)
    for r in range(R):
        for i in range(N // 8):
            word = 0
            for j in range(8):
                word |= int(codes[r, 8 * i + order[j]]) << (4 * j)
            out[r, i] = _i32(word)
    return torch.from_numpy(out.astype(np.int32))


def awq_dequant_shifts(qweight, qzeros, scales, G):
    """AWQ dequantisation by per-column shifts (column c of a word at bit
    shift (0, 16, 4, 20, 8, 24, 12, 28)[c]): an independent restatement."""
    shifts = [0, 16, 4, 20, 8, 24, 12, 28]
    qw = qweight.numpy().astype(np.int64) & 0xFFFFFFFF
    qz = qzeros.numpy().astype(np.int64) & 0xFFFFFFFF
    K, W = qw.shape
    N = W * 8
    out = np.zeros((K, N), dtype=np.float64)
    s = scales.numpy().astype(np.float64)
    for c in range(N):
        q = (qw[:, c // 8] >> shifts[c % 8]) & 0xF
        z = (qz[:, c // 8] >> shifts[c % 8]) & 0xF
        out[:, c] = (q - np.repeat(z, G)) * np.repeat(s[:, c], G)
    return out


def _rand(K, N, G, seed):
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    z = rng.integers(0, 16, size=(K // G, N), dtype=np.uint8)
    s = (rng.random((K // G, N)) * 9e-3 + 1e-3).astype(np.float16)
    return q, z, s


def test_gptq_worked_word():
    """One hand-made word: rows 0..7 of a column holding codes 1..8 -> 0x87654321."""
    q = np.zeros((8, 8), dtype=np.uint8)
    q[:, 3] = np.arange(1, 9)
    qw, _ = gptq_pack_loop(q, np.zeros((1, 8), dtype=np.uint8) + 1)
    assert int(qw[0, 3]) & 0xFFFFFFFF == 0x87654321
    assert F.gptq_codes(qw)[:, 3].tolist() == list(range(1, 9))


@pytest.mark.parametrize("zero_offset", [1, 0])
def test_gptq_without_act_order_matches_the_bit_loop(zero_offset):
    K, N, G = 64, 32, 16
    q, z, s = _rand(K, N, G, 1)
    qw, qz = gptq_pack_loop(q, z, zero_offset)
    w = F.gptq_to_tb(qw, qz, torch.from_numpy(s), torch.arange(K, dtype=torch.int32) // G, zero_offset)
    assert w.perm is None and w.group == G
    np.testing.assert_array_equal(w.packed.numpy(), oracle.pack_int4(q))
    np.testing.assert_array_equal(w.zeros.numpy(), oracle.pack_int4(z))
    back = F.tb_to_gptq(w, zero_offset)
    assert torch.equal(back[0], qw) and torch.equal(back[1], qz)


def test_gptq_act_order_permutation_preserves_the_product():
    """desc_act: g_idx assigns channels to groups out of order.  The converted
    weights with the activations permuted give the same product as the GPTQ
    definition W[k, n] = (q - z[g_idx[k]]) * s[g_idx[k]] on the original order."""
    K, N, G = 128, 16, 32
    rng = np.random.default_rng(2)
    q, z, s = _rand(K, N, G, 3)
    g_idx = (rng.permutation(K) // G).astype(np.int32)
    qw, qz = gptq_pack_loop(q, z)
    w = F.gptq_to_tb(qw, qz, torch.from_numpy(s), torch.from_numpy(g_idx))
    assert w.perm is not None
    W_ref = np.array([[(int(q[k, n]) - int(z[g_idx[k], n])) * float(s[g_idx[k], n]) for n in range(N)]
                      for k in range(K)])
    W_tb = oracle.int4_dequant(w.packed.numpy(), w.scales.numpy(), w.zeros.numpy(), G).astype(np.float64)
    A = rng.standard_normal((5, K))
    Ap = F.permute_input(torch.from_numpy(A), w.perm).numpy()
    np.testing.assert_allclose(Ap @ W_tb, A @ W_ref.astype(np.float16).astype(np.float64), rtol=1e-12, atol=1e-12)
    back = F.tb_to_gptq(w)
    assert torch.equal(back[0], qw) and torch.equal(back[1], qz) and back[3].tolist() == g_idx.tolist()


def test_gptq_rejects_unbalanced_groups():
    K, N, G = 64, 8, 16
    q, z, s = _rand(K, N, G, 4)
    qw, qz = gptq_pack_loop(q, z)
    g_idx = torch.arange(K) // G
    g_idx[0] = 1
    with pytest.raises(ValueError, match="exactly"):
        F.gptq_to_tb(qw, qz, torch.from_numpy(s), g_idx)


def test_awq_matches_bit_loop_and_shift_dequant():
    K, N, G = 64, 32, 32
    q, z, s = _rand(K, N, G, 5)
    qw, qz = awq_pack_loop(q), awq_pack_loop(z)
    w = F.awq_to_tb(qw, qz, torch.from_numpy(s))
    np.testing.assert_array_equal(w.packed.numpy(), oracle.pack_int4(q))
    np.testing.assert_array_equal(w.zeros.numpy(), oracle.pack_int4(z))
    W_tb = oracle.int4_dequant(w.packed.numpy(), w.scales.numpy(), w.zeros.numpy(), G).astype(np.float64)
    ref = awq_dequant_shifts(qw, qz, torch.from_numpy(s), G).astype(np.float16).astype(np.float64)
    np.testing.assert_array_equal(W_tb, ref)
    back = F.tb_to_awq(w)
    assert torch.equal(back[0], qw) and torch.equal(back[1], qz)


def _fnuz_value(c):
    """e4m3fnuz decoded from its definition: bias 8, no infinities, 0x80 NaN."""
    if c == 0x80:
        return float("nan")
    sign = -1.0 if c & 0x80 else 1.0
    e, m = (c >> 3) & 0xF, c & 7
    return sign * ((8 + m) * 2.0 ** (e - 11) if e else m * 2.0 ** -10)


def test_fp8_fnuz_checkpoint_reencoded_by_value():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    fw = F.fp8_checkpoint_to_tb(codes.view(torch.float8_e4m3fnuz).reshape(16, 16), weight_scale=0.5)
    out = oracle.e4m3_to_f32(fw.wqT.reshape(-1).numpy())
    inexact = []
    for c in range(256):
        v = _fnuz_value(c)
        if np.isnan(v):
            assert np.isnan(out[c])
        elif (v / 2.0 ** -9) == int(v / 2.0 ** -9):
            assert out[c] == v, (c, v, out[c])           # a multiple of fn's finest step: exact
        else:
            # an odd multiple of 2^-10 below 2^-6: halfway, rounded to the even multiple of 2^-9
            assert abs(out[c] - v) == 2.0 ** -10 and (abs(out[c]) / 2.0 ** -9) % 2 == 0, (c, v, out[c])
            inexact.append(c & 0x7F)
    assert sorted(set(inexact)) == [1, 3, 5, 7, 9, 11, 13, 15]
    assert torch.equal(fw.sw, torch.full((16,), 0.5))


def test_fp8_scale_conventions():
    W = torch.randn(6, 32).to(torch.float8_e4m3fn)
    per_ch = torch.rand(6, 1) + 0.5
    a = F.fp8_checkpoint_to_tb(W, per_ch)
    assert torch.equal(a.wqT, W.view(torch.uint8)) and torch.equal(a.sw, per_ch.reshape(6))
    # weight_scale_inv is the dequantisation multiplier too (DeepSeek-V3 / FineGrainedFP8)
    b = F.fp8_checkpoint_to_tb(W, weight_scale_inv=torch.tensor(4.0))
    assert torch.equal(b.sw, torch.full((6,), 4.0))
    with pytest.raises(ValueError, match="blocks"):
        F.fp8_checkpoint_to_tb(W, torch.ones(1, 1, 2))
    with pytest.raises(ValueError):
        F.fp8_checkpoint_to_tb(W)


def test_fp8_block_scales_select_the_block_gemm():
    """A DeepSeek-V3-style layer (weight [N, K], weight_scale_inv one fp32 per
    128 x 128 tile, ragged in N) converts to the block GEMM's operands, and
    dequantising through them is the reference's block map
    (weight_dequant: X * S[i//128, j//128])."""
    N, K = 300, 384
    g = torch.Generator().manual_seed(11)
    W = (torch.randn(N, K, generator=g) * 4).to(torch.float8_e4m3fn)
    inv = torch.rand(3, 3, generator=g) + 0.1
    f = F.fp8_checkpoint_to_tb(W, weight_scale_inv=inv)
    assert isinstance(f, F.Fp8BlockWeights) and f.block == 128
    assert torch.equal(f.wqT, W.view(torch.uint8)) and torch.equal(f.sw, inv)
    back = f.wqT.view(torch.float8_e4m3fn).to(torch.float32) * f.sw.repeat_interleave(128, 0)[:N].repeat_interleave(128, 1)
    ref = oracle.weight_dequant(W.to(torch.float32).numpy(), inv.numpy(), 128, "fp32")
    assert np.array_equal(back.numpy(), ref)
    with pytest.raises(ValueError, match="K % 128"):
        F.fp8_checkpoint_to_tb(torch.zeros(256, 200, dtype=torch.uint8), torch.ones(2, 2))
    # one K block: [ceil(N/128), 1] is still a block map when it is not [N, 1]
    f1 = F.fp8_checkpoint_to_tb(torch.zeros(256, 128, dtype=torch.uint8), torch.ones(2, 1))
    assert isinstance(f1, F.Fp8BlockWeights) and tuple(f1.sw.shape) == (2, 1)


def test_fp8_scale_inv_round_trip():
    """Quantise the way transformers' FineGrainedFP8 does (per output channel:
    q = w * 448 / amax, stored scale_inv = amax / 448) and dequantise through
    the converter's sw: the weight comes back to within e4m3's half step."""
    w = torch.randn(8, 64, generator=torch.Generator().manual_seed(5)) * 0.02
    amax = w.abs().amax(dim=1, keepdim=True)
    q = (w * (448.0 / amax)).to(torch.float8_e4m3fn)
    inv = amax / 448.0
    f = F.fp8_checkpoint_to_tb(q, weight_scale_inv=inv)
    back = f.wqT.view(torch.float8_e4m3fn).to(torch.float32) * f.sw[:, None]
    # e4m3 keeps 3 mantissa bits: relative error at most 2^-4 of each value
    assert torch.all((back - w).abs() <= w.abs() * 2.0 ** -4 + 1e-12)
    assert torch.allclose(back, w, rtol=0.07, atol=1e-4)


def test_safetensors_round_trip(tmp_path):
    from safetensors.torch import save_file

    K, N, G = 64, 16, 16
    q, z, s = _rand(K, N, G, 6)
    qw, qz = gptq_pack_loop(q, z)
    g_idx = torch.from_numpy((np.random.default_rng(7).permutation(K) // G).astype(np.int32))
    aw, az = awq_pack_loop(q), awq_pack_loop(z)
    W8 = torch.randn(N, K).to(torch.float8_e4m3fn)
    path = tmp_path / "model.safetensors"
    save_file({"l0.qweight": qw, "l0.qzeros": qz, "l0.scales": torch.from_numpy(s), "l0.g_idx": g_idx,
               "l1.qweight": aw, "l1.qzeros": az, "l1.scales": torch.from_numpy(s.copy()),
               "l2.weight": W8, "l2.weight_scale": torch.tensor([0.25])}, str(path))
    g = F.load_safetensors_layer(path, "l0", "gptq")
    ref = F.gptq_to_tb(qw, qz, torch.from_numpy(s), g_idx)
    assert torch.equal(g.packed, ref.packed) and torch.equal(g.perm, ref.perm)
    a = F.load_safetensors_layer(path, "l1", "awq")
    np.testing.assert_array_equal(a.packed.numpy(), oracle.pack_int4(q))
    f8 = F.load_safetensors_layer(path, "l2", "fp8")
    assert torch.equal(f8.wqT, W8.view(torch.uint8)) and torch.equal(f8.sw, torch.full((N,), 0.25))
    with pytest.raises(KeyError):
        F.load_safetensors_layer(path, "l9", "awq")


# ----------------------------------------------------------------------------- decode slab layout


def slab_byte_and_bit(k: int, n: int, K: int) -> tuple[int, int]:
    """Where code (k, n) lives in the slab layout, from the map's statement:
    slab s = n // 64, unit u = k // 32, lane l = 16 * ((k % 32) // 8) + n % 16,
    word b = (n % 64) // 16, code i = k % 8 at bit (i % 2) * 16 + (i // 2) * 4
    of that little-endian word."""
    s, u, i = n // 64, k // 32, k % 8
    lane = 16 * ((k % 32) // 8) + n % 16
    b = (n % 64) // 16
    bit = (i % 2) * 16 + (i // 2) * 4
    word_byte = ((s * (K // 32) + u) * 64 + lane) * 16 + 4 * b
    return word_byte + bit // 8, bit % 8


@pytest.mark.parametrize("k,n", [(0, 0), (1, 0), (7, 0), (8, 0), (31, 63), (32, 64), (5, 17), (100, 190), (127, 255)])
def test_slab_layout_places_single_codes(k, n):
    """A single non-zero code lands at the byte and bit the map names, and
    nowhere else (K = 128, N = 256)."""
    K, N = 128, 256
    q = np.zeros((K, N), np.uint8)
    q[k, n] = 0xB
    slabs = F.w4a16_to_slabs(F.pack_columns(torch.from_numpy(q)))
    assert tuple(slabs.shape) == F.slab_shape(K, N) == (N // 64, K // 32, 1024)
    flat = slabs.reshape(-1).numpy()
    byte, bit = slab_byte_and_bit(k, n, K)
    assert flat[byte] == 0xB << bit
    assert np.count_nonzero(flat) == 1


def test_slab_layout_round_trip_and_product():
    """Round trip to the packed layout is exact, and the torch reference
    gives the same product from either layout."""
    from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_torch
    from tilebench_amd.data import tensors as T

    A, p, s, z, G = T.generate_w4a16_gemm_inputs(3, 256, 192, 64, seed=9, device="cpu")
    slabs = F.w4a16_to_slabs(p)
    assert torch.equal(F.w4a16_from_slabs(slabs), p)
    assert torch.equal(impl_torch.run(A, slabs, s, z, G), impl_torch.run(A, p, s, z, G))
    A2, slabs2, s2, z2, _ = T.generate_w4a16_gemm_inputs(3, 256, 192, 64, seed=9, device="cpu", layout="slabs")
    assert torch.equal(slabs2, slabs) and torch.equal(A2, A)


def test_slab_layout_rejects_bad_shapes():
    with pytest.raises(ValueError):
        F.w4a16_to_slabs(torch.zeros(48, 32, dtype=torch.uint8))       # K % 32
    with pytest.raises(ValueError):
        F.w4a16_to_slabs(torch.zeros(64, 40, dtype=torch.uint8))       # N = 80, N % 64
    with pytest.raises(ValueError):
        from tilebench_amd.data import tensors as T
        T.generate_w4a16_gemm_inputs(17, 256, 128, 64, layout="slabs", device="cpu")
