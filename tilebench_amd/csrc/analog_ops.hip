// The reference's own dequantisation / quantisation operators on the hip
// backend (HBM-bound elementwise kernels):
//
//   weight_dequant      Y[i, j] = X[i, j] * S[i / T, j / T]         (fp16 / bf16 / fp32)
//   dequantize_rowwise  Y[r, c] = fp16((s[r] * x[r, c]) * (1 / 127)) (int8 -> fp16)
//   quantize_global     Y = fp16(x)                                  (fp32 -> fp16)
//
// Every product is formed in fp32 and rounded once to the output type (RNE),
// in the same order of operations as the PyTorch reference, so the results are
// bit-identical to it.  Each thread moves 16-byte vectors; consecutive threads
// take consecutive vectors of a row, so every wavefront access is contiguous.
#include "tb_common.h"

#pragma clang fp contract(off)

namespace tb {
namespace analog {

__device__ __forceinline__ float bf16_to_f(uint16_t h) { return __builtin_bit_cast(float, (uint32_t)h << 16); }

__device__ __forceinline__ uint16_t f_to_bf16(float f) {
  const uint32_t b = __builtin_bit_cast(uint32_t, f);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x40u);
  return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float h_to_f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f_to_h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// fp32 -> fp16 of a value that is itself a rounded fp32 product.  Without the
// empty asm the backend folds fptrunc(fmul) into v_fma_mixlo_f16, which rounds
// the exact product once to fp16; the reference rounds to fp32 first and then
// to fp16, and the two differ by one ulp on a few values in 10^4.
__device__ __forceinline__ uint16_t f_to_h_of_rounded(float f) {
  asm volatile("" : "+v"(f));
  return f_to_h(f);
}

// ---------------------------------------------------------------- weight_dequant
// One thread per 8 consecutive elements of a row (T % 8 == 0 keeps them in one
// scale tile).  DT: 0 fp32, 1 fp16, 2 bf16.
template <int DT>
__global__ void __launch_bounds__(256) weight_dequant_vec(const void* __restrict__ X, const void* __restrict__ S,
                                                          void* __restrict__ Y, int64_t M, int64_t N, int64_t T,
                                                          int64_t s_cols) {
  const int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_row = N >> 3;
  if (v >= M * per_row) return;
  const int64_t i = v / per_row, j = (v - i * per_row) * 8;
  const int64_t si = (i / T) * s_cols + j / T;
  if constexpr (DT == 0) {
    const float s = reinterpret_cast<const float*>(S)[si];
    const f32x4* x = reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(X) + i * N + j);
    f32x4* y = reinterpret_cast<f32x4*>(reinterpret_cast<float*>(Y) + i * N + j);
    const f32x4 a = __builtin_nontemporal_load(x), b = __builtin_nontemporal_load(x + 1);
    __builtin_nontemporal_store(a * s, y);
    __builtin_nontemporal_store(b * s, y + 1);
  } else {
    const uint16_t sb = reinterpret_cast<const uint16_t*>(S)[si];
    const float s = DT == 1 ? h_to_f(sb) : bf16_to_f(sb);
    const u32x4 xv = ld_nt(reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(X) + i * N + j));
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint16_t lo = (uint16_t)(xv[q] & 0xFFFFu), hi = (uint16_t)(xv[q] >> 16);
      const float a = (DT == 1 ? h_to_f(lo) : bf16_to_f(lo)) * s;
      const float b = (DT == 1 ? h_to_f(hi) : bf16_to_f(hi)) * s;
      o[q] = DT == 1 ? ((uint32_t)f_to_h(a) | ((uint32_t)f_to_h(b) << 16))
                     : ((uint32_t)f_to_bf16(a) | ((uint32_t)f_to_bf16(b) << 16));
    }
    st_nt(reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(Y) + i * N + j), o);
  }
}

template <int DT>
__global__ void __launch_bounds__(256) weight_dequant_scalar(const void* __restrict__ X, const void* __restrict__ S,
                                                             void* __restrict__ Y, int64_t M, int64_t N, int64_t T,
                                                             int64_t s_cols) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= M * N) return;
  const int64_t i = e / N, j = e - i * N;
  const int64_t si = (i / T) * s_cols + j / T;
  if constexpr (DT == 0) {
    reinterpret_cast<float*>(Y)[e] = reinterpret_cast<const float*>(X)[e] * reinterpret_cast<const float*>(S)[si];
  } else {
    const uint16_t xb = reinterpret_cast<const uint16_t*>(X)[e], sb = reinterpret_cast<const uint16_t*>(S)[si];
    const float p = DT == 1 ? h_to_f(xb) * h_to_f(sb) : bf16_to_f(xb) * bf16_to_f(sb);
    reinterpret_cast<uint16_t*>(Y)[e] = DT == 1 ? f_to_h(p) : f_to_bf16(p);
  }
}

// ---------------------------------------------------------------- dequantize_rowwise
// 16 int8 per thread -> 16 fp16 (two 16-byte stores).
__global__ void __launch_bounds__(256) dequant_rowwise_vec(const int8_t* __restrict__ x, const float* __restrict__ state,
                                                           uint16_t* __restrict__ y, int64_t rows, int64_t cols) {
  const int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_row = cols >> 4;
  if (v >= rows * per_row) return;
  const int64_t r = v / per_row, c = (v - r * per_row) * 16;
  const float s = state[r];
  const float inv127 = 1.0f / 127.0f;
  const u32x4 xv = ld_nt(reinterpret_cast<const u32x4*>(x + r * cols + c));
  u32x4 o[2];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int b = 0; b < 4; b += 2) {
      const float a0 = (s * (float)(int8_t)((xv[q] >> (8 * b)) & 0xFFu)) * inv127;
      const float a1 = (s * (float)(int8_t)((xv[q] >> (8 * (b + 1))) & 0xFFu)) * inv127;
      o[q >> 1][(q & 1) * 2 + (b >> 1)] = (uint32_t)f_to_h_of_rounded(a0) | ((uint32_t)f_to_h_of_rounded(a1) << 16);
    }
  }
  u32x4* dst = reinterpret_cast<u32x4*>(y + r * cols + c);
  st_nt(dst, o[0]);
  st_nt(dst + 1, o[1]);
}

// One row per blockIdx.y, 4096 elements per block: thread t converts elements
// t*8 .. t*8+7 and 2048 + t*8 .. +7 of the chunk, so each 8-byte load and each
// 16-byte store instruction of a wavefront covers one contiguous span (512 B
// read, 1 KiB written), and no thread divides to find its row.  Both loads go
// out before any branch (a lane past the row reads the row's first bytes and
// stores nothing), so they are in flight together.
__global__ void __launch_bounds__(256) dequant_rowwise_rows(const int8_t* __restrict__ x, const float* __restrict__ state,
                                                            uint16_t* __restrict__ y, int64_t cols) {
  const int64_t r = blockIdx.y;
  const float s = state[r];
  const float inv127 = 1.0f / 127.0f;
  int64_t c[2];
  u32x2 xv[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    c[h] = (int64_t)blockIdx.x * 4096 + h * 2048 + threadIdx.x * 8;
    // cols % 16 == 0: a thread's 8 elements are all in or all out
    xv[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(x + r * cols + (c[h] < cols ? c[h] : 0)));
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int b = 0; b < 4; b += 2) {
        const float a0 = (s * (float)(int8_t)((xv[h][q] >> (8 * b)) & 0xFFu)) * inv127;
        const float a1 = (s * (float)(int8_t)((xv[h][q] >> (8 * (b + 1))) & 0xFFu)) * inv127;
        o[q * 2 + (b >> 1)] = (uint32_t)f_to_h_of_rounded(a0) | ((uint32_t)f_to_h_of_rounded(a1) << 16);
      }
    if (c[h] < cols) st_nt(reinterpret_cast<u32x4*>(y + r * cols + c[h]), o);
  }
}

__global__ void __launch_bounds__(256) dequant_rowwise_scalar(const int8_t* __restrict__ x, const float* __restrict__ state,
                                                              uint16_t* __restrict__ y, int64_t rows, int64_t cols) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= rows * cols) return;
  const float inv127 = 1.0f / 127.0f;
  y[e] = f_to_h_of_rounded((state[e / cols] * (float)x[e]) * inv127);
}

// ---------------------------------------------------------------- quantize_global
// Groups of 4 elements; thread t of a block converts groups b*512 + t and
// b*512 + 256 + t, so each 16-byte load and each 8-byte store instruction of a
// wavefront covers one contiguous span.
__global__ void __launch_bounds__(256) f32_to_f16_vec(const f32x4* __restrict__ x, u32x2* __restrict__ y, int64_t n4) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t g = (int64_t)blockIdx.x * 512 + h * 256 + threadIdx.x;
    if (g >= n4) continue;
    const f32x4 a = __builtin_nontemporal_load(x + g);
    u32x2 o;
    o[0] = (uint32_t)f_to_h(a[0]) | ((uint32_t)f_to_h(a[1]) << 16);
    o[1] = (uint32_t)f_to_h(a[2]) | ((uint32_t)f_to_h(a[3]) << 16);
    __builtin_nontemporal_store(o, y + g);
  }
}

__global__ void __launch_bounds__(256) f32_to_f16_tail(const float* __restrict__ x, uint16_t* __restrict__ y,
                                                       int64_t start, int64_t n) {
  const int64_t e = start + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < n) y[e] = f_to_h(x[e]);
}

inline unsigned blocks_for(int64_t threads) { return (unsigned)((threads + 255) / 256); }

}  // namespace analog
}  // namespace tb

using namespace tb::analog;

extern "C" tb_status tb_weight_dequant(const void* X, const void* S, void* Y, int64_t M, int64_t N, int64_t tile,
                                       int dtype, hipStream_t stream) {
  TB_CHECK_ARG(X && S && Y, "tb_weight_dequant: null pointer");
  TB_CHECK_ARG(M > 0 && N > 0 && tile > 0, "tb_weight_dequant: M, N, TILE_SIZE must be positive");
  TB_CHECK_ARG(dtype >= 0 && dtype <= 2, "tb_weight_dequant: dtype must be 0 (fp32), 1 (fp16) or 2 (bf16)");
  TB_CHECK_ARG(M * N < (1ll << 40), "tb_weight_dequant: problem too large");
  const int64_t s_cols = (N + tile - 1) / tile;
  const bool vec = N % 8 == 0 && tile % 8 == 0 && tb::aligned(X, 16) && tb::aligned(Y, 16);
  const int64_t work = vec ? M * (N / 8) : M * N;
  TB_CHECK_ARG(work / 256 < (1ll << 31), "tb_weight_dequant: problem too large");
#define TB_WD_LAUNCH(D)                                                                                       \
  do {                                                                                                        \
    if (vec)                                                                                                  \
      hipLaunchKernelGGL(weight_dequant_vec<D>, dim3(blocks_for(work)), dim3(256), 0, stream, X, S, Y, M, N, \
                         tile, s_cols);                                                                       \
    else                                                                                                      \
      hipLaunchKernelGGL(weight_dequant_scalar<D>, dim3(blocks_for(work)), dim3(256), 0, stream, X, S, Y, M, \
                         N, tile, s_cols);                                                                    \
  } while (0)
  if (dtype == 0) TB_WD_LAUNCH(0);
  else if (dtype == 1) TB_WD_LAUNCH(1);
  else TB_WD_LAUNCH(2);
#undef TB_WD_LAUNCH
  return tb::launch_status("tb_weight_dequant");
}

extern "C" tb_status tb_dequantize_rowwise(const int8_t* x, const float* state, uint16_t* y, int64_t rows,
                                           int64_t cols, hipStream_t stream) {
  TB_CHECK_ARG(x && state && y, "tb_dequantize_rowwise: null pointer");
  TB_CHECK_ARG(rows > 0 && cols > 0 && rows * cols < (1ll << 40), "tb_dequantize_rowwise: bad shape");
  const bool vec = cols % 16 == 0 && tb::aligned(x, 16) && tb::aligned(y, 16);
  if (vec && rows <= 65535)
    hipLaunchKernelGGL(dequant_rowwise_rows, dim3((unsigned)((cols + 4095) / 4096), (unsigned)rows), dim3(256), 0,
                       stream, x, state, y, cols);
  else if (vec)
    hipLaunchKernelGGL(dequant_rowwise_vec, dim3(blocks_for(rows * (cols / 16))), dim3(256), 0, stream, x, state, y,
                       rows, cols);
  else
    hipLaunchKernelGGL(dequant_rowwise_scalar, dim3(blocks_for(rows * cols)), dim3(256), 0, stream, x, state, y, rows,
                       cols);
  return tb::launch_status("tb_dequantize_rowwise");
}

extern "C" tb_status tb_quantize_global(const float* x, uint16_t* y, int64_t n, hipStream_t stream) {
  TB_CHECK_ARG(x && y && n > 0 && n < (1ll << 40), "tb_quantize_global: bad arguments");
  int64_t done = 0;
  if (tb::aligned(x, 16) && tb::aligned(y, 16) && n >= 8) {
    const int64_t n4 = n / 8 * 2;
    hipLaunchKernelGGL(f32_to_f16_vec, dim3((unsigned)((n4 + 511) / 512)), dim3(256), 0, stream,
                       reinterpret_cast<const tb::f32x4*>(x), reinterpret_cast<tb::u32x2*>(y), n4);
    done = n4 * 4;
  }
  if (done < n)
    hipLaunchKernelGGL(f32_to_f16_tail, dim3(blocks_for(n - done)), dim3(256), 0, stream, x, y, done, n);
  return tb::launch_status("tb_quantize_global");
}
