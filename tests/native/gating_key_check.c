/* The gating filter kernel's key maps (tilebench_amd/csrc/moe_gating.hip):
 * key_of_bits (any fp32 pattern) and key_of_finite (no NaN check, used on
 * rows known to be finite).  Checks, over every fp32 bit pattern:
 *   1. key_of_finite(b) == key_of_bits(b) for every finite b;
 *   2. key order is float order on finite values with -0 == +0: walking the
 *      finite values from -max to +max, keys rise by exactly one per step,
 *      except the step from -0 to +0, where they are equal.
 * Built with -DPLANT_DROPPED_SUBTRACT the finite map loses its "- s" term and
 * the program must report mismatches. */
#include <stdint.h>
#include <stdio.h>

static uint32_t key_of_bits(uint32_t b) {
  const uint32_t mag = b & 0x7FFFFFFFu;
  const uint32_t neg = (uint32_t)((int32_t)b >> 31);
  const uint32_t key = 0x80000000u + ((mag ^ neg) - neg);
  return mag > 0x7F800000u ? 0xFFFFFFFFu : key;
}

static uint32_t key_of_finite(uint32_t b) {
  const uint32_t sm = (uint32_t)((int32_t)b >> 31);
#ifdef PLANT_DROPPED_SUBTRACT
  return b ^ (sm | 0x80000000u);
#else
  return (b ^ (sm | 0x80000000u)) - sm;
#endif
}

int main(void) {
  uint64_t mismatches = 0, order_errors = 0, checked = 0;
#pragma omp parallel for reduction(+ : mismatches, checked)
  for (int64_t x = 0; x < (int64_t)(1ull << 32); ++x) {
    const uint32_t b = (uint32_t)x;
    if (((b >> 23) & 0xFFu) == 0xFFu) continue;  /* inf / NaN */
    ++checked;
    if (key_of_finite(b) != key_of_bits(b)) ++mismatches;
  }
  /* increasing finite values: negative magnitudes from max down to 0, then positive ones up */
  uint32_t prev = key_of_finite(0xFF7FFFFFu);
  for (int64_t m = 0x7F7FFFFE; m >= 0; --m) {
    const uint32_t k = key_of_finite(0x80000000u | (uint32_t)m);
    if (k != prev + 1) ++order_errors;
    prev = k;
  }
  for (uint32_t m = 0; m <= 0x7F7FFFFFu; ++m) {
    const uint32_t k = key_of_finite(m);
    if (k != (m == 0 ? prev : prev + 1)) ++order_errors;
    prev = k;
  }
  printf("checked=%llu mismatches=%llu order_errors=%llu\n", (unsigned long long)checked,
         (unsigned long long)mismatches, (unsigned long long)order_errors);
  return (mismatches || order_errors) ? 1 : 0;
}
