// Shared device/host helpers for libtbhip (gfx950 / CDNA4 only).
//
// Everything here is written for 64-lane wavefronts. Host-side helpers record
// a thread-local error message that tb_last_error() returns; entry points never
// print, abort or allocate device memory.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "tbhip.h"

namespace tb {

// ---------------------------------------------------------------- host errors
void set_error(const char* fmt, ...);

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

#define TB_CHECK_ARG(cond, ...)                         \
  do {                                                  \
    if (!(cond)) {                                      \
      ::tb::set_error(__VA_ARGS__);                     \
      return TB_E_INVALID;                              \
    }                                                   \
  } while (0)

#define TB_CHECK_ALIGN(ptr, a, name)                                                    \
  do {                                                                                  \
    if (!::tb::aligned((ptr), (a))) {                                                   \
      ::tb::set_error("%s must be %d-byte aligned (got %p)", (name), (int)(a), (ptr));  \
      return TB_E_ALIGN;                                                                \
    }                                                                                   \
  } while (0)

// Allow `kernel` up to `bytes` of dynamic LDS on the current device.  The
// attribute is set once per (kernel, device) pair (a process may drive several
// GPUs); thread-safe.
tb_status reserve_lds(const void* kernel, size_t bytes, const char* what);

// Report the status of the launch that was just enqueued.
inline tb_status launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return TB_E_HIP;
  }
  return TB_OK;
}

// ------------------------------------------------------------- device helpers
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Non-temporal 16-byte global load/store: streamed data is read once, so it
// should not evict reused data (scales, zero-points) from L2.
__device__ __forceinline__ u32x4 ld_nt(const u32x4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_nt(u32x4* p, u32x4 v) { __builtin_nontemporal_store(v, p); }

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Raw buffer resource over `bytes` bytes at p: loads through it at offsets past
// the end return zeros without touching memory, so a load can be issued for
// every lane, with an out-of-range offset where there is nothing to read,
// instead of sitting behind a per-lane branch.
typedef __amdgpu_buffer_rsrc_t buf_rsrc_t;
constexpr uint32_t BUF_OOB = 0x80000000u;
__device__ __forceinline__ buf_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ uint32_t as_u32(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// Two int4 codes (in bytes 0 and 2 of `pair`, values 0..15) to a half2 holding
// 1024 + code: 0x6400 is 1024.0 in fp16 and its ulp is 1, so OR-ing the code
// into the mantissa is an exact conversion.
__device__ __forceinline__ f16x2 magic_h2(uint32_t pair) { return as_h2(pair | 0x64006400u); }

// fp32 -> OCP fp8-e4m3 code, round to nearest even, no saturation: magnitudes
// at or above 480 (whose rounding would need the reserved S.1111.111 pattern),
// inf and NaN give the NaN code 0x7F with the sign kept, as torch's
// float -> float8_e4m3fn cast does.  Subnormals (below 2^-6) round onto the
// 2^-9 grid through one fp32 addition of 2^14, whose ulp is 2^-9.
__device__ __forceinline__ uint32_t e4m3_code(float q) {
  uint32_t b = __builtin_bit_cast(uint32_t, q);
  const uint32_t sign = (b >> 24) & 0x80u;
  b &= 0x7FFFFFFFu;
  uint32_t c;
  if (b >= 0x43F00000u) {
    c = 0x7Fu;
  } else if (b < (121u << 23)) {
    const float t = __builtin_bit_cast(float, b) + 16384.0f;
    c = __builtin_bit_cast(uint32_t, t) - (141u << 23);
  } else {
    c = (b + 0xC407FFFFu + ((b >> 20) & 1u)) >> 20;  // 0xC407FFFF = (-120 << 23) + 0x7FFFF (mod 2^32)
  }
  return (c | sign) & 0xFFu;
}

// fp32 -> bf16 bits, round to nearest even, NaN kept quiet.
__device__ __forceinline__ uint32_t bf16_bits(float f) {
  const uint32_t b = __builtin_bit_cast(uint32_t, f);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (b >> 16) | 0x40u;
  return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

}  // namespace tb
