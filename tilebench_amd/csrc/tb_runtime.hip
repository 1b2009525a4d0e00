// Library-level entry points: version, error reporting, the cache-flush fill
// kernel and the HBM streaming-copy probe.
#include "tb_common.h"

#include <string.h>

#include <mutex>

namespace tb {

static thread_local char g_last_error[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

tb_status reserve_lds(const void* kernel, size_t bytes, const char* what) {
  struct Entry {
    const void* kernel;
    int device;
  };
  static std::mutex mu;
  static Entry done[256];
  static int n_done = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    set_error("%s: no current device", what);
    return TB_E_HIP;
  }
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < n_done; ++i)
    if (done[i].kernel == kernel && done[i].device == dev) return TB_OK;
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) != hipSuccess) {
    set_error("%s: cannot reserve %zu bytes of LDS", what, bytes);
    return TB_E_HIP;
  }
  if (n_done < 256) done[n_done++] = Entry{kernel, dev};  // past 256 pairs the attribute is simply set again
  return TB_OK;
}

// Streaming kernels are written one 16-byte granule per thread over a grid
// that covers the whole buffer: on MI355X that shape sustains 6.7 TB/s for a
// 512 MiB copy, where grid-stride loops (2048-8192 blocks, four granules in
// flight per thread) reach 4.7-5.1 TB/s and eight granules per thread 4.3 TB/s.
//
// The flush uses plain (cache-allocating) stores: nontemporal stores leave the
// MALL's contents in place (a 64 MiB buffer read back after a 1 GiB
// nontemporal fill is exactly as fast as without it), plain stores of 384 MiB
// or more evict it (profiles/mall_sweep_MI355X.txt).
__global__ void __launch_bounds__(256) fill_kernel(u32x4* __restrict__ dst, int64_t n16, uint32_t pattern) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n16) dst[i] = u32x4{pattern, pattern, pattern, pattern};
}

// Streaming copy, one 16-byte granule per thread (see fill_kernel).
__global__ void __launch_bounds__(256) copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                   int64_t n16) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n16) st_nt(dst + i, ld_nt(src + i));
}

// Streaming read, one 16-byte granule per thread, plain (cache-allocating)
// loads: the re-read probe of the eviction sweep.  The XOR of what a thread
// read is stored only if it equals a key no input holds, so the loads stay
// live without writing anything.
__global__ void __launch_bounds__(256) read_kernel(const u32x4* __restrict__ src, int64_t n16, uint32_t key,
                                                   uint32_t* __restrict__ sink) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n16) {
    const u32x4 v = src[i];
    const uint32_t x = v[0] ^ v[1] ^ v[2] ^ v[3];
    if (x == key) sink[0] = x;
  }
}

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// MFMA throughput probe: every wavefront keeps 8 independent 32x32 accumulators
// busy for `iters` rounds, so the matrix pipe never waits on a dependency; the
// accumulators are reduced to one store per lane so nothing is dead code.
// kind 0: v_mfma_f32_32x32x16_f16 (32768 flop), kind 1: v_mfma_f32_32x32x64_f8f6f4
// with e4m3 operands (131072 flop), kind 2: v_mfma_f32_32x32x16_bf16 (32768 flop),
// kind 3: v_mfma_i32_32x32x32_i8 (65536 op).
template <int KIND>
__global__ void __launch_bounds__(256) mfma_probe_kernel(float* __restrict__ out, int iters, float seed) {
  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f32x16{};
  const int lane = threadIdx.x;
  if constexpr (KIND == 0) {
    h8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[i] = (_Float16)(seed * (lane + i));
      b[i] = (_Float16)(seed * (lane - i));
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[i], 0, 0, 0);
    }
  } else if constexpr (KIND == 2) {
    bf8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[i] = (__bf16)(seed * (lane + i));
      b[i] = (__bf16)(seed * (lane - i));
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[i], 0, 0, 0);
    }
  } else if constexpr (KIND == 3) {
    i32x16 iacc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) iacc[i] = i32x16{};
    i32x4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = (int)(0x01020304u * (uint32_t)(lane + i + 1));
      b[i] = (int)(0x04030201u * (uint32_t)(lane - i + 7));
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 8; ++i) iacc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, iacc[i], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][e] = (float)iacc[i][e];
  } else {
    i32x8 a, b;  // e4m3 codes 0x30..0x37 (0.25 .. 0.4375) and 0x28..0x2F (0.0625 .. 0.109)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[i] = (int)(0x30303030u + (uint32_t)((lane + i) & 7));
      b[i] = (int)(0x28282828u + (uint32_t)((lane ^ i) & 7));
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        acc[i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc[i], 0, 0, 0, 0, 0, 0);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[i][e];
  out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Clock probe: the fp16 loop of mfma_probe_kernel<0> between two reads of the
// shader clock counter (s_memtime) and of the constant 100 MHz counter
// (s_memrealtime).  Thread 0 of block b writes both differences to
// clocks[2 b] and clocks[2 b + 1], so the host reads the block's average
// shader clock as 100 MHz x the ratio; every wavefront's first lane writes a
// sum of its accumulators to sink[4 b + wave] (so no MFMA is dead code).
__global__ void __launch_bounds__(256) clock_probe_kernel(unsigned long long* __restrict__ clocks,
                                                          float* __restrict__ sink, int iters, float seed) {
  const uint64_t c0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f32x16{};
  const int lane = threadIdx.x;
  h8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (_Float16)(seed * (lane + i));
    b[i] = (_Float16)(seed * (lane - i));
  }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[i], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[i][e];
  const uint64_t c1 = __builtin_amdgcn_s_memtime();
  const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
  if ((threadIdx.x & 63) == 0) sink[(int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)] = s;
  if (threadIdx.x == 0) {
    clocks[2 * (int64_t)blockIdx.x] = c1 - c0;
    clocks[2 * (int64_t)blockIdx.x + 1] = r1 - r0;
  }
}

static unsigned grid_for(int64_t n16) { return (unsigned)((n16 + 255) / 256); }

}  // namespace tb

extern "C" {

const char* tb_version(void) { return "tbhip 0.1.0 gfx950"; }

const char* tb_last_error(void) { return tb::g_last_error; }

tb_status tb_l2_flush(void* buf, int64_t bytes, uint32_t pattern, hipStream_t stream) {
  TB_CHECK_ARG(buf != nullptr && bytes > 0 && bytes % 16 == 0, "tb_l2_flush: bytes must be a positive multiple of 16");
  TB_CHECK_ARG(bytes / 16 / 256 < (1ll << 31), "tb_l2_flush: buffer too large");
  TB_CHECK_ALIGN(buf, 16, "buf");
  const int64_t n16 = bytes / 16;
  hipLaunchKernelGGL(tb::fill_kernel, dim3(tb::grid_for(n16)), dim3(256), 0, stream,
                     reinterpret_cast<tb::u32x4*>(buf), n16, pattern);
  return tb::launch_status("tb_l2_flush");
}

tb_status tb_probe_mfma(int kind, int64_t blocks, int64_t iters, float* out, hipStream_t stream) {
  TB_CHECK_ARG(out != nullptr && blocks > 0 && blocks < (1 << 24) && iters > 0 && iters < (1 << 30),
               "tb_probe_mfma: bad arguments");
  TB_CHECK_ARG(kind >= 0 && kind <= 3, "tb_probe_mfma: kind must be 0 (fp16), 1 (fp8), 2 (bf16) or 3 (int8)");
  const dim3 grid((unsigned)blocks), block(256);
  if (kind == 0)
    hipLaunchKernelGGL(tb::mfma_probe_kernel<0>, grid, block, 0, stream, out, (int)iters, 1e-3f);
  else if (kind == 1)
    hipLaunchKernelGGL(tb::mfma_probe_kernel<1>, grid, block, 0, stream, out, (int)iters, 1e-3f);
  else if (kind == 2)
    hipLaunchKernelGGL(tb::mfma_probe_kernel<2>, grid, block, 0, stream, out, (int)iters, 1e-3f);
  else
    hipLaunchKernelGGL(tb::mfma_probe_kernel<3>, grid, block, 0, stream, out, (int)iters, 1e-3f);
  return tb::launch_status("tb_probe_mfma");
}

tb_status tb_probe_clock(int64_t blocks, int64_t iters, uint64_t* clocks, float* sink, hipStream_t stream) {
  TB_CHECK_ARG(clocks && sink && blocks > 0 && blocks < (1ll << 31) && iters > 0 && iters < (1ll << 31),
               "tb_probe_clock: bad arguments");
  TB_CHECK_ALIGN(clocks, 8, "clocks");
  hipLaunchKernelGGL(tb::clock_probe_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     reinterpret_cast<unsigned long long*>(clocks), sink, (int)iters, 1e-3f);
  return tb::launch_status("tb_probe_clock");
}

tb_status tb_probe_read(const void* src, int64_t bytes, uint32_t key, uint32_t* sink, hipStream_t stream) {
  TB_CHECK_ARG(src && sink && bytes > 0 && bytes % 16 == 0, "tb_probe_read: bytes must be a positive multiple of 16");
  TB_CHECK_ARG(bytes / 16 / 256 < (1ll << 31), "tb_probe_read: buffer too large");
  TB_CHECK_ALIGN(src, 16, "src");
  TB_CHECK_ALIGN(sink, 4, "sink");
  const int64_t n16 = bytes / 16;
  hipLaunchKernelGGL(tb::read_kernel, dim3(tb::grid_for(n16)), dim3(256), 0, stream,
                     reinterpret_cast<const tb::u32x4*>(src), n16, key, sink);
  return tb::launch_status("tb_probe_read");
}

tb_status tb_probe_copy(const void* src, void* dst, int64_t bytes, hipStream_t stream) {
  TB_CHECK_ARG(src && dst && bytes > 0 && bytes % 16 == 0, "tb_probe_copy: bytes must be a positive multiple of 16");
  TB_CHECK_ARG(bytes / 16 / 256 < (1ll << 31), "tb_probe_copy: buffer too large");
  TB_CHECK_ALIGN(src, 16, "src");
  TB_CHECK_ALIGN(dst, 16, "dst");
  const int64_t n16 = bytes / 16;
  hipLaunchKernelGGL(tb::copy_kernel, dim3(tb::grid_for(n16)), dim3(256), 0, stream,
                     reinterpret_cast<const tb::u32x4*>(src), reinterpret_cast<tb::u32x4*>(dst), n16);
  return tb::launch_status("tb_probe_copy");
}

}  // extern "C"
