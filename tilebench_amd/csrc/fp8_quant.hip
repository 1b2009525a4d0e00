// Per-token fp8-e4m3 activation quantisation (HBM-bound).
//
//   sa[m]    = fp32(max_k |A[m,k]|) / 448            (IEEE division)
//   Aq[m,k]  = e4m3(RN32(fp32(A[m,k]) / sa[m]))      (RNE, no saturation)
//
// One 256-thread block per row.  The row is read from HBM once: each thread
// keeps its ITEMS 16-byte chunks (8 halfs each) in registers while the block
// reduces the absolute maximum (packed u16 max on the sign-cleared bits, which
// orders finite fp16 magnitudes exactly, then a wavefront shuffle reduction
// and a 4-entry LDS exchange).
//
// Division.  Per element the quotient x / sa is formed as
//   q0 = RN(x * y) with y = RN(1 / sa) computed once per row by an IEEE divide,
//   r  = fma(-q0, sa, x)   (exact remainder),   q = RN(q0 + r * y)  (fma),
// with the sign of x copied onto q (keeps -0.0), the reciprocal-refinement scheme of Markstein (IBM J. Res. Dev. 34(1), 1990).
// Its agreement with the IEEE quotient is not assumed: the whole input domain
// of this kernel (every finite fp16 row maximum times every fp16 x with
// |x| <= max) is checked exhaustively on the CPU by the test suite.
//
// Conversion to e4m3 (OCP "fn": bias 7, 3 mantissa bits, max 448, no infinity,
// S.1111.111 = NaN).  Finite, non-zero rows use the hardware converter
// v_cvt_pk_fp8_f32 (their quotients lie in [-448, 448], where it rounds exactly
// like the encoder below; see quantize_chunk).  Rows with inf or NaN use the
// integer encoder e4m3_code (tb_common.h), which rounds to nearest-even on the
// magnitude bits:
//   |q| >= 480 (0x43F00000)      -> 0x7F (NaN code), sign OR-ed back in
//   |q| <  2^-6 (subnormal range) -> add 2^14 in fp32: the sum's ulp is 2^-9, the
//                                   e4m3 subnormal step, so the hardware RNE add
//                                   rounds to the right multiple; subtract the
//                                   bits of 2^14 to get the code (0..8)
//   otherwise                     -> rebias the exponent (-120 << 23) and round
//                                   the 20 dropped mantissa bits to nearest-even
//                                   with the +0x7FFFF + lsb trick; a carry into
//                                   the exponent is the correct rounding result
//                                   (448 < |q| <= 464 rounds to 448, above -> NaN)
#include "tb_common.h"
#include "fp8_codec.h"

#pragma clang fp contract(off)

namespace tb {

template <int ITEMS>
__global__ void __launch_bounds__(256) fp8_quant_rows(const u32x4* __restrict__ A, u32x2* __restrict__ Aq,
                                                      float* __restrict__ sa_out, int64_t K) {
  __shared__ uint32_t red[4];
  const int64_t row = blockIdx.x;
  const int64_t chunks = K >> 3;  // 8 halfs per 16-byte chunk
  const u32x4* src = A + row * chunks;

  // Every chunk is a buffer load, chunks past the row end reading zeros (which
  // leave the maximum unchanged): no branch around a load, so all of a
  // thread's loads are in flight together.
  const buf_rsrc_t rs = buf_rsrc(src, (uint32_t)(chunks * 16));
  u32x4 x[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int64_t ch = threadIdx.x + (int64_t)i * 256;
    x[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, ch < chunks ? (uint32_t)(ch * 16) : BUF_OOB, 0, 2 /* nt */);
  }
  uint32_t m = 0;  // packed pair of u16 magnitudes
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t a = x[i][j] & 0x7FFF7FFFu;
      m = max(m & 0xFFFFu, a & 0xFFFFu) | (max(m >> 16, a >> 16) << 16);
    }
  m = max(m & 0xFFFFu, m >> 16);
  m = wave_max_u32(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = max(max(red[0], red[1]), max(red[2], red[3]));

  const float amax = (float)__builtin_bit_cast(_Float16, (uint16_t)m);
  const float sa = amax / 448.0f;
  const float y = 1.0f / sa;
  if (threadIdx.x == 0) sa_out[row] = sa;

#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int64_t ch = threadIdx.x + (int64_t)i * 256;
    if (ch < chunks) Aq[row * chunks + ch] = quantize_chunk(x[i], sa, y, m);
  }
}

// Rows longer than 256 * 8 * 8 halfs: two passes over the row (the second
// one is served by L2).
__global__ void __launch_bounds__(256) fp8_quant_rows_long(const u32x4* __restrict__ A, u32x2* __restrict__ Aq,
                                                           float* __restrict__ sa_out, int64_t K) {
  __shared__ uint32_t red[4];
  const int64_t row = blockIdx.x;
  const int64_t chunks = K >> 3;
  const u32x4* src = A + row * chunks;
  uint32_t m = 0;
  for (int64_t ch = threadIdx.x; ch < chunks; ch += 256) {
    const u32x4 v = src[ch];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t a = v[j] & 0x7FFF7FFFu;
      m = max(m, max(a & 0xFFFFu, a >> 16));
    }
  }
  m = wave_max_u32(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = max(max(red[0], red[1]), max(red[2], red[3]));
  const float amax = (float)__builtin_bit_cast(_Float16, (uint16_t)m);
  const float sa = amax / 448.0f;
  const float y = 1.0f / sa;
  if (threadIdx.x == 0) sa_out[row] = sa;
  for (int64_t ch = threadIdx.x; ch < chunks; ch += 256) Aq[row * chunks + ch] = quantize_chunk(src[ch], sa, y, m);
}

}  // namespace tb

extern "C" tb_status tb_fp8_act_quant(const uint16_t* A, uint8_t* Aq, float* sa, int64_t M, int64_t K,
                                      hipStream_t stream) {
  TB_CHECK_ARG(A && Aq && sa, "tb_fp8_act_quant: null pointer");
  TB_CHECK_ARG(M > 0 && K > 0 && K % 8 == 0, "tb_fp8_act_quant: need M > 0 and K a positive multiple of 8 (M=%lld K=%lld)",
               (long long)M, (long long)K);
  TB_CHECK_ARG(M < (1ll << 31), "tb_fp8_act_quant: M too large");
  TB_CHECK_ALIGN(A, 16, "A");
  TB_CHECK_ALIGN(Aq, 8, "Aq");
  const auto* a = reinterpret_cast<const tb::u32x4*>(A);
  auto* q = reinterpret_cast<tb::u32x2*>(Aq);
  const int64_t chunks = K / 8;
  const dim3 grid((unsigned)M), block(256);
  if (chunks <= 256) hipLaunchKernelGGL(tb::fp8_quant_rows<1>, grid, block, 0, stream, a, q, sa, K);
  else if (chunks <= 512) hipLaunchKernelGGL(tb::fp8_quant_rows<2>, grid, block, 0, stream, a, q, sa, K);
  else if (chunks <= 1024) hipLaunchKernelGGL(tb::fp8_quant_rows<4>, grid, block, 0, stream, a, q, sa, K);
  else if (chunks <= 2048) hipLaunchKernelGGL(tb::fp8_quant_rows<8>, grid, block, 0, stream, a, q, sa, K);
  else hipLaunchKernelGGL(tb::fp8_quant_rows_long, grid, block, 0, stream, a, q, sa, K);
  return tb::launch_status("tb_fp8_act_quant");
}
