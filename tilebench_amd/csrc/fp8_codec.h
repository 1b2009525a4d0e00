// fp8-e4m3 quantisation of fp16 values by a positive fp32 scale, shared by
// the per-token and the per-token-block quantisers (device code, gfx950).
#pragma once

#include "tb_common.h"

namespace tb {

// The refinement yields +0 for x = -0 (fma(+0, y, -0) = +0); sa and y are
// positive, so the quotient always carries the sign of x and copysign restores it.
__device__ __forceinline__ float quotient(float x, float sa, float y) {
#pragma clang fp contract(off)
  const float q0 = x * y;
  const float r = __builtin_fmaf(-q0, sa, x);
  return __builtin_copysignf(__builtin_fmaf(r, y, q0), x);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off, 64));
  return v;
}

// Eight fp16 values -> eight e4m3 codes of x / sa.  `m` is the row's largest
// magnitude as fp16 bits.  For a finite, non-zero row every quotient lies in
// [-448, 448] (up to one fp32 rounding), where the hardware conversion
// v_cvt_pk_fp8_f32 rounds exactly as the integer encoder e4m3_code (checked on
// the device against the torch-pinned CPU oracle for all e4m3 values, every
// rounding midpoint +-1 fp32 ulp, the subnormal range, signed zeros and 3*10^6
// random values with |x| <= 464: no difference).
//
// The other rows follow the IEEE quotient with the NaN results of the x86
// vector divide that the CPU reference runs (an invalid operation gives the
// default NaN, sign set; a NaN operand propagates, the dividend's first):
//   zero row (sa = 0):        0 / 0 is invalid             -> 0xFF
//   row max inf (sa = inf):   finite x / inf = +-0          -> 0x00 / 0x80,
//                             +-inf / inf is invalid       -> 0xFF
//   row holds NaN (sa = NaN): a NaN x propagates its sign   -> 0x7F | sign(x),
//                             any other x gets sa's NaN (a magnitude, positive) -> 0x7F
__device__ __forceinline__ u32x2 quantize_chunk(const u32x4& x, float sa, float y, uint32_t m) {
  u32x2 o;
  if (m == 0) {
    o[0] = o[1] = 0xFFFFFFFFu;
  } else if (m < 0x7C00u) {
    float q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint16_t h = (uint16_t)((x[j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
      q[j] = quotient((float)__builtin_bit_cast(_Float16, h), sa, y);
    }
    o[0] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
    o[0] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], (int)o[0], true);
    o[1] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
    o[1] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], (int)o[1], true);
  } else {
    uint32_t c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t h = (x[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
      const uint32_t sign = (h >> 8) & 0x80u, mag = h & 0x7FFFu;
      if (m > 0x7C00u)
        c[j] = mag > 0x7C00u ? (0x7Fu | sign) : 0x7Fu;
      else
        c[j] = mag == 0x7C00u ? 0xFFu : sign;
    }
    o[0] = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
    o[1] = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
  }
  return o;
}

}  // namespace tb
