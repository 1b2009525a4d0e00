"""numpy restatement of the hot-path operators (test infrastructure only).

Every function works on host numpy arrays.  fp16 is numpy float16; bf16 and
fp8-e4m3 are carried as their raw uint16 / uint8 bit patterns.
"""
from __future__ import annotations

import numpy as np

# ----------------------------------------------------------------------------- int4 packing


def pack_int4(q: np.ndarray) -> np.ndarray:
    """uint8 codes [..., C] in [0, 15] -> uint8 [..., C/2], low nibble first:
    byte j = q[2j] | q[2j+1] << 4 (the BASELINE config-0 packing)."""
    q = np.asarray(q, dtype=np.uint8)
    if q.shape[-1] % 2:
        raise ValueError("last dimension must be even")
    if (q > 15).any():
        raise ValueError("int4 codes must be in [0, 15]")
    return (q[..., 0::2] | (q[..., 1::2] << 4)).astype(np.uint8)


def unpack_int4(p: np.ndarray) -> np.ndarray:
    """Inverse of pack_int4: uint8 [..., C/2] -> uint8 codes [..., C]."""
    p = np.asarray(p, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p & 0x0F
    out[..., 1::2] = p >> 4
    return out


# ----------------------------------------------------------------------------- int4 dequant


def int4_dequant(packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray, group: int) -> np.ndarray:
    """fp16 [K, N] = fp16((q - z) * s), groups of `group` rows along K.

    packed uint8 [K, N/2]; scales fp16 [K/G, N]; zeros uint8 [K/G, N/2] (packed
    like the weights).  (q - z) is an exact small integer and its product with an
    fp16 scale is exact in fp32, so the only rounding is the final fp32 -> fp16
    (round-to-nearest-even, which numpy's astype implements)."""
    q = unpack_int4(packed).astype(np.int16)
    z = unpack_int4(zeros).astype(np.int16)
    K, N = q.shape
    if K % group:
        raise ValueError("K must be a multiple of the group size")
    s = np.asarray(scales, dtype=np.float16).astype(np.float32)
    if s.shape != (K // group, N) or z.shape != (K // group, N):
        raise ValueError("scales / zeros must be [K/G, N]")
    d = (q.reshape(K // group, group, N) - z[:, None, :]).astype(np.float32)
    with np.errstate(over="ignore"):  # products past the fp16 range round to inf, as the cast defines
        return (d * s[:, None, :]).astype(np.float16).reshape(K, N)


# ----------------------------------------------------------------------------- bf16 helpers


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern, round-to-nearest-even; NaN -> quiet NaN."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r[nan] = ((b[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------- fp8 e4m3


def e4m3_from_f32(x: np.ndarray) -> np.ndarray:
    """fp32 -> OCP fp8-e4m3 ("fn") codes, round-to-nearest-even, no saturation.

    Magnitudes at or above 480 (the first value whose rounding would need the
    reserved S.1111.111 pattern) and NaN/inf give the NaN code 0x7F; the sign
    bit is kept.  Values below 2^-6 round onto the subnormal grid 2^-9 * m."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    sign = ((b >> 24) & 0x80).astype(np.uint8)
    mag = b & np.uint32(0x7FFFFFFF)
    out = np.empty(mag.shape, dtype=np.uint8)

    nan = mag >= np.uint32(0x43F00000)
    sub = mag < np.uint32(121 << 23)
    nrm = ~(nan | sub)

    out[nan] = 0x7F
    # subnormal grid: round |x| / 2^-9 to the nearest integer, ties to even
    # (exact in float64: |x| < 2^-6 has at most 24 significant bits)
    v = mag[sub].view(np.float32).astype(np.float64) * 512.0
    out[sub] = np.rint(v).astype(np.uint8)  # np.rint rounds half to even
    # normal range: keep 3 mantissa bits, RNE on the 20 dropped bits, rebias 127 -> 7
    m = mag[nrm].astype(np.uint64)
    kept = m >> 20
    rem = m & 0xFFFFF
    up = (rem > 0x80000) | ((rem == 0x80000) & ((kept & 1) == 1))
    code = kept + up.astype(np.uint64) - (120 << 3)
    out[nrm] = code.astype(np.uint8)
    return out | sign


_E4M3_TABLE = None


def e4m3_to_f32(c: np.ndarray) -> np.ndarray:
    """fp8-e4m3 codes -> fp32 values (exact)."""
    global _E4M3_TABLE
    if _E4M3_TABLE is None:
        t = np.empty(256, dtype=np.float32)
        for code in range(256):
            s = -1.0 if code & 0x80 else 1.0
            e = (code >> 3) & 0xF
            m = code & 7
            if e == 15 and m == 7:
                t[code] = np.nan
            elif e == 0:
                t[code] = s * m * 2.0 ** -9
            else:
                t[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
        _E4M3_TABLE = t
    return _E4M3_TABLE[np.asarray(c, dtype=np.uint8)]


def fp8_act_quant(A: np.ndarray):
    """Per-row fp8 quantisation of fp16 A [M, K] -> (codes uint8 [M, K], sa fp32 [M]).

    sa = fp32(max |A[m]|) / 448; codes = e4m3(fp32(A) / sa), both IEEE fp32
    divisions.  An all-zero row has sa = 0 and every code 0xFF (the NaN with the
    sign bit that x86 produces for 0/0)."""
    A = np.asarray(A, dtype=np.float16)
    amax = np.abs(A).max(axis=1).astype(np.float32)
    sa = (amax / np.float32(448.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = (A.astype(np.float32) / sa[:, None]).astype(np.float32)
    codes = e4m3_from_f32(q)
    codes[amax == 0] = 0xFF
    return codes, sa


def fp8_scaled_gemm(Aq: np.ndarray, Wq: np.ndarray, sa: np.ndarray, sw: np.ndarray) -> np.ndarray:
    """Y bf16 bits [M, N] = bf16(sa[m] * sw[n] * sum_k e4m3(Aq[m,k]) * e4m3(Wq[k,n])).

    Aq [M, K] and Wq [K, N] are e4m3 codes (any strides).  The product of two
    e4m3 values is exact in float64 and K <= 2^16 terms of it sum with error far
    below the bf16 rounding, so this is the fp32-accumulate result rounded once."""
    a = e4m3_to_f32(Aq).astype(np.float64)
    w = e4m3_to_f32(Wq).astype(np.float64)
    acc = a @ w
    y = (acc * np.asarray(sa, np.float64)[:, None]) * np.asarray(sw, np.float64)[None, :]
    return f32_to_bf16_bits(y.astype(np.float32))


def fp8_act_quant_blocks(A: np.ndarray, block: int = 128):
    """Per-token, per-block fp8 quantisation of fp16 A [M, K] (K % block == 0)
    -> (codes uint8 [M, K], sa fp32 [K/block, M], block-major).

    Each block of `block` consecutive elements of a row is quantised exactly as
    fp8_act_quant quantises a row: sa = fp32(max |block|) / 448, codes =
    e4m3(fp32(A) / sa), an all-zero block giving sa = 0 and 0xFF codes."""
    A = np.asarray(A, dtype=np.float16)
    M, K = A.shape
    if K % block:
        raise ValueError(f"K = {K} is not a multiple of the block size {block}")
    codes, sa = fp8_act_quant(A.reshape(M * (K // block), block))
    return codes.reshape(M, K), np.ascontiguousarray(sa.reshape(M, K // block).T)


def fp8_block_gemm(Aq: np.ndarray, WqT: np.ndarray, sa: np.ndarray, sw: np.ndarray, block: int = 128) -> np.ndarray:
    """Y bf16 bits [M, N] = bf16( sum_kb s[kb, m, n] * P_kb[m, n] ) with
    P_kb = sum_{k in block kb} e4m3(Aq[m,k]) * e4m3(WqT[n,k]) and
    s = fp32(sa[kb, m] * sw[n // block, kb]).

    Aq [M, K] and WqT [N, K] are e4m3 codes, sa fp32 [K/block, M], sw fp32
    [ceil(N/block), K/block].  Each P_kb is exact in float64 (128 products of
    4-bit significands spanning at most 2^-18 .. 2^18); the scaled terms are
    summed in float64 in block order and the sum is rounded once to bf16."""
    a = e4m3_to_f32(Aq).astype(np.float64)
    w = e4m3_to_f32(WqT).astype(np.float64)
    M, K = a.shape
    N = w.shape[0]
    sa = np.asarray(sa, np.float32)
    sw = np.asarray(sw, np.float32)
    nkb = K // block
    if K % block or sa.shape != (nkb, M) or sw.shape != ((N + block - 1) // block, nkb):
        raise ValueError("fp8_block_gemm: operand / scale shapes do not match")
    col_block = np.arange(N) // block
    acc = np.zeros((M, N), np.float64)
    for kb in range(nkb):
        ks = slice(kb * block, (kb + 1) * block)
        P = a[:, ks] @ w[:, ks].T
        s = (sa[kb][:, None] * sw[col_block, kb][None, :]).astype(np.float32)
        acc += s.astype(np.float64) * P
    return f32_to_bf16_bits(acc.astype(np.float32))


# ----------------------------------------------------------------------------- W4A16 GEMMs


def w4a16_gemm(A: np.ndarray, packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray, group: int) -> np.ndarray:
    """fp16 [M, N] = fp16(A @ dequant(W)) with fp32 accumulation."""
    W = int4_dequant(packed, scales, zeros, group).astype(np.float32)
    return (np.asarray(A, dtype=np.float16).astype(np.float32) @ W).astype(np.float16)


def moe_w4a16_grouped_gemm(A: np.ndarray, packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray,
                           offsets: np.ndarray, group: int) -> np.ndarray:
    """Grouped W4A16: rows offsets[e]:offsets[e+1] of A use expert e's weights.

    A fp16 [R, K]; packed uint8 [E, K, N/2]; scales fp16 [E, K/G, N]; zeros uint8
    [E, K/G, N/2]; offsets int [E+1], non-decreasing, offsets[0] = 0,
    offsets[E] = R.  Returns fp16 [R, N]."""
    E = packed.shape[0]
    off = np.asarray(offsets, dtype=np.int64)
    if off.shape != (E + 1,) or off[0] != 0 or off[-1] != A.shape[0] or (np.diff(off) < 0).any():
        raise ValueError("offsets must be [E+1], non-decreasing, from 0 to R")
    N = packed.shape[2] * 2
    Y = np.zeros((A.shape[0], N), dtype=np.float16)
    for e in range(E):
        lo, hi = off[e], off[e + 1]
        if hi > lo:
            Y[lo:hi] = w4a16_gemm(A[lo:hi], packed[e], scales[e], zeros[e], group)
    return Y


# ----------------------------------------------------------------------------- MoE gating


def moe_topk_gating(logits: np.ndarray, k: int, dtype: str = "fp32"):
    """Top-k gating of logits [M, E] -> (weights [M, k], indices int32 [M, k]).

    Order: logits descending, NaN above everything, equal logits (including
    -0.0 == +0.0) by ascending expert index.  Weights: softmax over the k
    selected logits in fp32, returned in the logits' dtype.  `dtype` is "fp32",
    "fp16" or "bf16"; bf16 logits and weights are uint16 bit patterns."""
    if dtype == "bf16":
        x = bf16_bits_to_f32(logits)
    else:
        x = np.asarray(logits).astype(np.float32)
    M, E = x.shape
    if not 1 <= k <= E:
        raise ValueError("need 1 <= k <= E")
    idx = np.broadcast_to(np.arange(E), (M, E))
    isnan = np.isnan(x)
    v = np.where(isnan, 0.0, x).astype(np.float64) + 0.0  # + 0.0 folds -0.0 onto +0.0
    order = np.lexsort((idx, -v, ~isnan), axis=-1)[:, :k]
    vals = np.take_along_axis(x, order, axis=1).astype(np.float32)
    with np.errstate(invalid="ignore"):  # rows holding inf - inf or NaN give NaN weights (IEEE arithmetic)
        e = np.exp(vals - vals[:, :1]).astype(np.float32)
        w = (e / e.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)
    if dtype == "fp16":
        w = w.astype(np.float16)
    elif dtype == "bf16":
        w = f32_to_bf16_bits(w)
    return w, order.astype(np.int32)


# ----------------------------------------------------------------------------- MoE layer


def moe_align(topk_ids: np.ndarray, experts: int):
    """(token, slot) pair ids p = t * topk + j (the flattened index of
    topk_ids [T, k]) ordered by expert and, within an expert, by p; ids outside
    [0, E) are routed nowhere.  Returns (sorted_ids int32 [n_valid], offsets
    int32 [E + 1]), offsets[e] = number of pairs with an id below e."""
    flat = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    valid = (flat >= 0) & (flat < experts)
    pid = np.nonzero(valid)[0]
    order = np.argsort(flat[pid], kind="stable")
    counts = np.bincount(flat[pid], minlength=experts)
    offsets = np.zeros(experts + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts)
    return pid[order].astype(np.int32), offsets.astype(np.int32)


def silu_mul(h: np.ndarray) -> np.ndarray:
    """fp16 [R, I] = fp16(silu(g) * u) of fp16 h [R, 2I] = [g | u] (gate in the
    first half), silu(x) = x / (1 + exp(-x)), every step in fp32."""
    h = np.asarray(h, dtype=np.float16)
    I = h.shape[-1] // 2
    g = h[..., :I].astype(np.float32)
    u = h[..., I:].astype(np.float32)
    with np.errstate(over="ignore"):   # exp(-g) and the fp16 cast may overflow to inf, as on the device
        den = (np.float32(1.0) + np.exp(-g)).astype(np.float32)
        return ((g / den).astype(np.float32) * u).astype(np.float16)


def moe_gate_up(X: np.ndarray, sorted_ids: np.ndarray, offsets: np.ndarray, topk: int, packed: np.ndarray,
                scales: np.ndarray, zeros: np.ndarray, group: int) -> np.ndarray:
    """Sorted row m of expert e reads token sorted_ids[m] // topk of X fp16
    [T, H]; act [n_valid, I] = silu_mul(fp16(X[t] @ dequant(W13_e))) with
    W13 int4 [E, H, 2I] (packed [E, H, I], scales [E, H/G, 2I], zeros
    [E, H/G, I])."""
    E = packed.shape[0]
    I = packed.shape[2]
    act = np.zeros((len(sorted_ids), I), dtype=np.float16)
    tok = np.asarray(sorted_ids, dtype=np.int64) // topk
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi > lo:
            act[lo:hi] = silu_mul(w4a16_gemm(X[tok[lo:hi]], packed[e], scales[e], zeros[e], group))
    return act


def moe_down(act: np.ndarray, sorted_ids: np.ndarray, offsets: np.ndarray, weights: np.ndarray, pairs: int,
             packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray, group: int):
    """Y [pairs, H] fp16: row sorted_ids[m] = fp16(w[sorted_ids[m]] * fp32(act[m]
    @ dequant(W2_e))) (the fp32 product rounded once, to fp16, after the
    weight), W2 int4 [E, I, H].  Returns (Y, written), `written` marking the
    rows a pair of a valid expert produced (the kernel leaves the others)."""
    E = packed.shape[0]
    H = packed.shape[2] * 2
    Y = np.zeros((pairs, H), dtype=np.float16)
    written = np.zeros(pairs, dtype=bool)
    w = np.asarray(weights, dtype=np.float32).reshape(-1)
    sid = np.asarray(sorted_ids, dtype=np.int64)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi > lo:
            Wd = int4_dequant(packed[e], scales[e], zeros[e], group).astype(np.float32)
            acc = (act[lo:hi].astype(np.float32) @ Wd).astype(np.float32)
            rows = sid[lo:hi]
            Y[rows] = (acc * w[rows][:, None]).astype(np.float32).astype(np.float16)
            written[rows] = True
    return Y, written


def moe_combine(Y: np.ndarray, topk_ids: np.ndarray, experts: int) -> np.ndarray:
    """out fp16 [T, H] = fp16(sum over slots j in order of fp32(Y[t * k + j])),
    slots routed nowhere skipped."""
    ids = np.asarray(topk_ids)
    T, k = ids.shape
    valid = (ids >= 0) & (ids < experts)
    Yr = Y.reshape(T, k, -1)
    acc = np.zeros((T, Yr.shape[2]), dtype=np.float32)
    for j in range(k):
        acc = np.where(valid[:, j:j + 1], (acc + Yr[:, j].astype(np.float32)).astype(np.float32), acc)
    return acc.astype(np.float16)


def fused_moe_w4a16(X, logits, W13, S13, Z13, W2, S2, Z2, topk: int, group13: int, group2: int) -> np.ndarray:
    """The MoE layer: gating of fp32 logits [T, E] (moe_topk_gating), align,
    gate/up with SiLU * up, down scaled by the routing weight, combine."""
    T, E = np.asarray(logits).shape
    w, ids = moe_topk_gating(np.asarray(logits, dtype=np.float32), topk, "fp32")
    sid, off = moe_align(ids, E)
    act = moe_gate_up(np.asarray(X, dtype=np.float16), sid, off, topk, W13, S13, Z13, group13)
    Y, _ = moe_down(act, sid, off, w, T * topk, W2, S2, Z2, group2)
    return moe_combine(Y, ids, E)


# ----------------------------------------------------------------------------- reference analog operators


def weight_dequant(X: np.ndarray, S: np.ndarray, tile: int, dtype: str = "fp16") -> np.ndarray:
    """Y[i, j] = X[i, j] * S[i // T, j // T] in the tensors' dtype ("fp32", "fp16",
    or "bf16" with uint16 bit patterns): the product of two such values is exact
    in fp32, then rounded once to the dtype."""
    if dtype == "bf16":
        x, s = bf16_bits_to_f32(X), bf16_bits_to_f32(S)
    else:
        x, s = np.asarray(X).astype(np.float32), np.asarray(S).astype(np.float32)
    M, N = x.shape
    full = np.repeat(np.repeat(s, tile, axis=0)[:M], tile, axis=1)[:, :N]
    y = (x * full).astype(np.float32)
    if dtype == "fp16":
        return y.astype(np.float16)
    if dtype == "bf16":
        return f32_to_bf16_bits(y)
    return y


def dequantize_rowwise(x: np.ndarray, state: np.ndarray) -> np.ndarray:
    """fp16((state[r] * x[r, c]) * (1/127)), two fp32 roundings then one to fp16."""
    prod = (np.asarray(state, np.float32)[:, None] * np.asarray(x).astype(np.float32)).astype(np.float32)
    return (prod * np.float32(1.0 / 127.0)).astype(np.float32).astype(np.float16)


def quantize_global(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16, round to nearest even (overflow -> inf)."""
    with np.errstate(over="ignore"):
        return np.asarray(x, np.float32).astype(np.float16)


# ----------------------------------------------------------------------------- plain GEMM operators


def unpack_i2(b: np.ndarray, K: int) -> np.ndarray:
    """uint8 [K/4, N] with four 2-bit fields per byte -> int8 [K, N]: row
    i*K/4 + kb is ((b[kb] >> 2i) & 3) - 1 (matmul_int8/impl_torch.py:10-14)."""
    b = np.asarray(b, dtype=np.uint8)
    Kb = b.shape[0]
    if K != 4 * Kb:
        raise ValueError("A's K dim must be 4x B's K_b dim")
    return np.concatenate([((b >> (2 * i)) & 3).astype(np.int8) - 1 for i in range(4)], axis=0)


def matmul_int8(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """int32 [M, N] = a int8 [M, K] @ unpack_i2(b), exact (matmul_int8/impl_torch.py:4-19,
    whose fp32 matmul is exact for these ranges: |sum| < 2^24)."""
    a = np.asarray(a, dtype=np.int8)
    B = unpack_i2(b, a.shape[1])
    # every partial sum is an integer below 2^53 in magnitude, so float64 BLAS is exact
    return np.rint(a.astype(np.float64) @ B.astype(np.float64)).astype(np.int64).astype(np.int32)


def matmul_f16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """fp16 [M, N] = fp16(a @ b), products and sum in float64 (the reference's
    fp32-accumulated torch.matmul differs from it by accumulation rounding only)."""
    return (np.asarray(a, np.float16).astype(np.float64) @ np.asarray(b, np.float16).astype(np.float64)).astype(np.float16)


def matmul_f32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """fp32 [M, N] = a @ b in float64, rounded once."""
    return (np.asarray(a, np.float32).astype(np.float64) @ np.asarray(b, np.float32).astype(np.float64)).astype(np.float32)


def matmul_fp8(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """e4m3 codes [M, N] = e4m3(bf16(a @ b)) for e4m3 code operands a [M, K],
    b [K, N]: the reference's _scaled_mm with unit scales and bf16 output, then
    .to(float8_e4m3fn) (matmul_fp32_fp16_fp8/impl_torch.py:21-26).  Products of
    e4m3 values are exact in float64."""
    acc = e4m3_to_f32(a).astype(np.float64) @ e4m3_to_f32(b).astype(np.float64)
    y16 = bf16_bits_to_f32(f32_to_bf16_bits(acc.astype(np.float32)))
    return e4m3_from_f32(y16)
