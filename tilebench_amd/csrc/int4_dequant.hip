// Int4 group-wise weight dequantisation (HBM-bound).
//
// out[k, n] = fp16((q[k, n] - z[k/G, n]) * s[k/G, n]) with q, z int4 codes in
// the N-packed, low-nibble-first layout (byte [k, j] = q[k,2j] | q[k,2j+1] << 4).
//
// Vector path: one thread owns 32 consecutive columns (one 16-byte packed load
// per row) over ROWS consecutive rows of one group.  Its scales (64 B) and
// zero-points (16 B) are loaded once and kept in registers as half2 pairs; each
// row then costs one 16-byte load and four 16-byte stores, all coalesced
// across the wavefront.  Codes become fp16 through the 0x6400 magic number
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
__global__ void __launch_bounds__(256) int4_dequant_vec(const u32x4* __restrict__ packed,
                                                        const u32x4* __restrict__ scales,
                                                        const u32x4* __restrict__ zeros,
                                                        u32x4* __restrict__ out, int64_t K, int64_t N,
                                                        int64_t group) {
  const int64_t chunks = N >> 5;  // 32-column chunks per row
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t c = tid % chunks;
  const int64_t r0 = (tid / chunks) * ROWS;
  if (r0 >= K) return;
  const int64_t g = r0 / group;

  // Zero-points of the 32 columns: 16 bytes -> 16 half2 of (1024 + z).
  f16x2 zh[16];
  {
    const u32x4 zw = zeros[g * chunks + c];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f16x2 t[4];
      unpack8(zw[i], t);
#pragma unroll
      for (int j = 0; j < 4; ++j) zh[4 * i + j] = t[j];
    }
  }
  // Scales of the 32 columns: 64 bytes -> 16 half2.
  f16x2 sh[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 sw = scales[(g * chunks + c) * 4 + i];
#pragma unroll
    for (int j = 0; j < 4; ++j) sh[4 * i + j] = as_h2(sw[j]);
  }

  u32x4 w[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) w[r] = ld_nt(packed + (r0 + r) * chunks + c);

#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    u32x4* dst = out + ((r0 + r) * chunks + c) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f16x2 h[4];
      unpack8(w[r][i], h);
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = as_u32((h[j] - zh[4 * i + j]) * sh[4 * i + j]);
      st_nt(dst + i, o);
    }
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
  constexpr int ROWS = 4;
  const bool vec = (N % 32 == 0) && (group % ROWS == 0) && tb::aligned(packed, 16) && tb::aligned(scales, 16) &&
                   tb::aligned(zeros, 16) && tb::aligned(out, 16);
  if (vec) {
    const int64_t threads = (N / 32) * (K / ROWS);
    const int64_t blocks = (threads + 255) / 256;
    TB_CHECK_ARG(blocks < (1ll << 31), "tb_int4_dequant: problem too large");
    hipLaunchKernelGGL(tb::int4_dequant_vec<ROWS>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       reinterpret_cast<const tb::u32x4*>(packed), reinterpret_cast<const tb::u32x4*>(scales),
                       reinterpret_cast<const tb::u32x4*>(zeros), reinterpret_cast<tb::u32x4*>(out), K, N, group);
  } else {
    const int64_t blocks = (K * (N / 2) + 255) / 256;
    TB_CHECK_ARG(blocks < (1ll << 31), "tb_int4_dequant: problem too large");
    hipLaunchKernelGGL(tb::int4_dequant_scalar, dim3((unsigned)blocks), dim3(256), 0, stream, packed, scales, zeros,
                       out, K, N, group);
  }
  return tb::launch_status("tb_int4_dequant");
}
