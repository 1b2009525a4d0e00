/*
 * Exhaustive CPU check of the fp8 quantiser's division scheme (test suite only).
 *
 * The kernel tb_fp8_act_quant forms x / sa as
 *     y = RN(1 / sa);  q0 = RN(x * y);  r = fma(-q0, sa, x);  q = copysign(RN(q0 + r*y), x)
 * and must agree with the IEEE quotient RN(x / sa) bit for bit.  Every case the
 * kernel can meet is enumerated: sa = RN(amax / 448) for every positive finite
 * fp16 row maximum amax, and every fp16 x with |x| <= amax (both signs).
 * fp32 multiply, divide and fmaf are IEEE operations on the CPU and on gfx950
 * alike (no denormal fp32 values occur: |x / sa| >= 2^-24 / (65504/448)).
 *
 * Prints "pairs=<n> mismatches=<m>" and exits 0 only if m == 0.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float h2f(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  uint32_t b;
  if (e == 0) {
    if (m == 0) {
      b = s;
    } else { /* subnormal: m * 2^-24, exact in fp32 */
      float f = (float)m * 0x1p-24f;
      memcpy(&b, &f, 4);
      b |= s;
    }
  } else if (e == 31) {
    b = s | 0x7F800000u | (m << 13);
  } else {
    b = s | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &b, 4);
  return f;
}

static uint32_t bits(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}

int main(void) {
  unsigned long long pairs = 0, bad = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : pairs, bad)
  for (int a = 1; a < 0x7C00; ++a) {
    const float amax = h2f((uint16_t)a);
    volatile float sa_v = amax / 448.0f;
    const float sa = sa_v;
    volatile float y_v = 1.0f / sa;
    const float y = y_v;
    for (int xb = 0; xb <= a; ++xb) {
      for (int sgn = 0; sgn < 2; ++sgn) {
        const float x = h2f((uint16_t)(xb | (sgn << 15)));
        volatile float ref_v = x / sa;
        const float q0 = x * y;
        const float r = fmaf(-q0, sa, x);
#ifdef PLANT_DROPPED_COPYSIGN /* the test suite's planted mistake: must be detected */
        const float q = fmaf(r, y, q0);
#else
        const float q = copysignf(fmaf(r, y, q0), x);
#endif
        pairs++;
        if (bits(q) != bits(ref_v)) {
          bad++;
        }
      }
    }
  }
  printf("pairs=%llu mismatches=%llu\n", pairs, bad);
  return bad == 0 ? 0 : 1;
}
