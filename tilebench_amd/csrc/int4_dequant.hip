// Int4 group-wise weight dequantisation (HBM-bound).
//
// out[k, n] = fp16((q[k, n] - z[k/G, n]) * s[k/G, n]) with q, z int4 codes in
// the N-packed, low-nibble-first layout (byte [k, j] = q[k,2j] | q[k,2j+1] << 4).
//
// Vector path: a lane owns 8 consecutive columns (one packed dword per row)
// over ROWS consecutive rows of one group; consecutive lanes own consecutive
// column groups, so every wavefront-wide load (4 B per lane) and store (16 B
// per lane, 8 fp16) covers one contiguous span of a row.  The lane's 8 scales
// (16 B) and 8 zero-points (4 B) are loaded once per ROWS rows and kept in
// registers as half2 pairs.  Codes become fp16 through the 0x6400 magic number
// (1024 + q, exact), the zero-point subtraction is exact, and the single
// rounding is the half2 multiply by the scale (RNE), so the result is
// bit-identical to fp16(float(q - z) * float(s)).
#include "tb_common.h"

#pragma clang fp contract(off)

namespace tb {

// Expand one packed dword (8 codes, columns c..c+7) into 4 half2 pairs of
// (1024 + q) holding columns (c, c+1), (c+2, c+3), ...
__device__ __forceinline__ void unpack8(uint32_t w, f16x2 (&h)[4]) {
  const uint32_t even = w & 0x0F0F0F0Fu;         // codes of columns c, c+2, c+4, c+6
  const uint32_t odd = (w >> 4) & 0x0F0F0F0Fu;   // codes of columns c+1, c+3, c+5, c+7
  // perm(odd, even, sel): bytes 0-3 address `even`, 4-7 address `odd`, 0x0C -> 0.
  h[0] = magic_h2(perm(odd, even, 0x0C040C00u));
  h[1] = magic_h2(perm(odd, even, 0x0C050C01u));
  h[2] = magic_h2(perm(odd, even, 0x0C060C02u));
  h[3] = magic_h2(perm(odd, even, 0x0C070C03u));
}

template <int ROWS>
__global__ void __launch_bounds__(256) int4_dequant_vec(const uint32_t* __restrict__ packed,
                                                        const u32x4* __restrict__ scales,
                                                        const uint32_t* __restrict__ zeros,
                                                        u32x4* __restrict__ out, int64_t K, int64_t N,
                                                        int64_t group) {
  const int64_t cgs = N >> 3;  // 8-column groups per row
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t c = tid % cgs;
  const int64_t r0 = (tid / cgs) * ROWS;
  if (r0 >= K) return;
  const int64_t g = r0 / group;

  uint32_t w[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) w[r] = __builtin_nontemporal_load(packed + (r0 + r) * cgs + c);

  f16x2 zh[4], sh[4];
  unpack8(zeros[g * cgs + c], zh);
  const u32x4 sw = scales[g * cgs + c];
#pragma unroll
  for (int j = 0; j < 4; ++j) sh[j] = as_h2(sw[j]);

#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    f16x2 h[4];
    unpack8(w[r], h);
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = as_u32((h[j] - zh[j]) * sh[j]);
    st_nt(out + (r0 + r) * cgs + c, o);
  }
}

// Any even N: one thread per packed byte (two output columns).
__global__ void __launch_bounds__(256) int4_dequant_scalar(const uint8_t* __restrict__ packed,
                                                           const uint16_t* __restrict__ scales,
                                                           const uint8_t* __restrict__ zeros,
                                                           uint16_t* __restrict__ out, int64_t K, int64_t N,
                                                           int64_t group) {
  const int64_t half_n = N >> 1;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= K * half_n) return;
  const int64_t k = i / half_n, j = i % half_n, g = k / group;
  const uint32_t b = packed[i], zb = zeros[g * half_n + j];
  const f16x2 h = magic_h2((b & 0xFu) | ((b >> 4) << 16));
  const f16x2 zh = magic_h2((zb & 0xFu) | ((zb >> 4) << 16));
  const uint32_t s = scales[g * N + 2 * j] | ((uint32_t)scales[g * N + 2 * j + 1] << 16);
  const uint32_t o = as_u32((h - zh) * as_h2(s));
  out[k * N + 2 * j] = (uint16_t)(o & 0xFFFFu);
  out[k * N + 2 * j + 1] = (uint16_t)(o >> 16);
}

}  // namespace tb

extern "C" tb_status tb_int4_dequant(const uint8_t* packed, const uint16_t* scales, const uint8_t* zeros,
                                     uint16_t* out, int64_t K, int64_t N, int64_t group,
                                     hipStream_t stream) {
  TB_CHECK_ARG(packed && scales && zeros && out, "tb_int4_dequant: null pointer");
  TB_CHECK_ARG(K > 0 && N > 0 && group > 0, "tb_int4_dequant: K, N, group must be positive (K=%lld N=%lld G=%lld)",
               (long long)K, (long long)N, (long long)group);
  TB_CHECK_ARG(N % 2 == 0, "tb_int4_dequant: N must be even (got %lld)", (long long)N);
  TB_CHECK_ARG(K % group == 0, "tb_int4_dequant: K=%lld is not a multiple of group=%lld", (long long)K,
               (long long)group);
  constexpr int ROWS = 8;
  const bool vec = (N % 8 == 0) && (group % ROWS == 0) && tb::aligned(packed, 16) && tb::aligned(scales, 16) &&
                   tb::aligned(zeros, 16) && tb::aligned(out, 16);
  if (vec) {
    const int64_t threads = (N / 8) * (K / ROWS);
    const int64_t blocks = (threads + 255) / 256;
    TB_CHECK_ARG(blocks < (1ll << 31), "tb_int4_dequant: problem too large");
    hipLaunchKernelGGL(tb::int4_dequant_vec<ROWS>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       reinterpret_cast<const uint32_t*>(packed), reinterpret_cast<const tb::u32x4*>(scales),
                       reinterpret_cast<const uint32_t*>(zeros), reinterpret_cast<tb::u32x4*>(out), K, N, group);
  } else {
    const int64_t blocks = (K * (N / 2) + 255) / 256;
    TB_CHECK_ARG(blocks < (1ll << 31), "tb_int4_dequant: problem too large");
    hipLaunchKernelGGL(tb::int4_dequant_scalar, dim3((unsigned)blocks), dim3(256), 0, stream, packed, scales, zeros,
                       out, K, N, group);
  }
  return tb::launch_status("tb_int4_dequant");
}
