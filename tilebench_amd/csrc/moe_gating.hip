// MoE router gating: per row, top-k logits (descending, equal logits -> lowest
// expert index first) and the softmax over those k logits in fp32.
//
// Layout: a block stages ROWS consecutive rows of logits in LDS with one
// coalesced 16-byte sweep (the rows are contiguous in HBM), converting each
// logit to an order-preserving uint32 key on the way in.  Each row is then
// owned by LPR lanes (a power of two, consecutive lanes), each holding V keys
// of that row in registers.  k selection rounds follow: every lane takes its
// largest remaining key (ascending index order, strict '>', so the lowest index
// wins a tie), the LPR lanes combine (key, index) pairs with xor-shuffles, and
// the owner of the winner clears it.  Selection runs on the logits themselves,
// never on exp() values, so rounding in exp cannot create or break ties.
//
// Key map: k(x) = bits ^ 0x80000000 for x >= 0 and ~bits for x < 0, with -0.0
// folded onto +0.0 (they compare equal) and every NaN mapped to 0xFFFFFFFF (a
// NaN ranks above +inf, as in torch.topk).  Real keys are >= k(-inf) =
// 0x007FFFFF, so 0 marks a taken (or absent) slot.
#include "tb_common.h"

namespace tb {

__device__ __forceinline__ uint32_t key_of_bits(uint32_t b) {
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return 0xFFFFFFFFu;  // NaN
  if (b == 0x80000000u) b = 0;                             // -0.0 == +0.0
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float float_of_key(uint32_t u) {
  const uint32_t b = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
  return __builtin_bit_cast(float, b);
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays a quiet NaN).
__device__ __forceinline__ uint16_t bf16_rne(float f) {
  const uint32_t b = __builtin_bit_cast(uint32_t, f);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x40u);
  return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

template <int DT>
__device__ __forceinline__ uint32_t load_key(const void* base, int64_t i) {
  if constexpr (DT == 0) {
    return key_of_bits(reinterpret_cast<const uint32_t*>(base)[i]);
  } else if constexpr (DT == 1) {
    const uint16_t h = reinterpret_cast<const uint16_t*>(base)[i];
    return key_of_bits(__builtin_bit_cast(uint32_t, (float)__builtin_bit_cast(_Float16, h)));
  } else {
    const uint16_t h = reinterpret_cast<const uint16_t*>(base)[i];
    return key_of_bits((uint32_t)h << 16);
  }
}

template <int DT>
__device__ __forceinline__ void store_weight(void* base, int64_t i, float w) {
  if constexpr (DT == 0) {
    reinterpret_cast<float*>(base)[i] = w;
  } else if constexpr (DT == 1) {
    reinterpret_cast<uint16_t*>(base)[i] = __builtin_bit_cast(uint16_t, (_Float16)w);
  } else {
    reinterpret_cast<uint16_t*>(base)[i] = bf16_rne(w);
  }
}

constexpr int kBlock = 256;
constexpr int kPad = 4;  // LDS row padding (dwords) against bank conflicts
constexpr int kBatch = 8;  // 16-byte loads in flight per thread while staging

template <int DT, int V, int LPR, int KMAX>
__global__ void __launch_bounds__(kBlock) gating_kernel(const void* __restrict__ logits, void* __restrict__ weights,
                                                        int32_t* __restrict__ indices, int64_t M, int E, int k) {
  constexpr int ROWS = kBlock / LPR;
  extern __shared__ uint32_t lds[];
  const int stride = E + kPad;
  const int64_t row0 = (int64_t)blockIdx.x * ROWS;
  const int nrows = (int)((M - row0) < ROWS ? (M - row0) : ROWS);

  // Stage the block's rows (contiguous in HBM) as keys.  Loads are issued in
  // batches of kBatch independent 16-byte loads per thread before any of them
  // is consumed, so one HBM round trip covers a batch.
  {
    const int64_t base = row0 * E;
    const int total = nrows * E;
    constexpr int EPV = DT == 0 ? 4 : 8;  // elements per 16-byte vector
    if ((E % EPV) == 0) {
      const u32x4* src = reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(logits) +
                                                        base * (DT == 0 ? 4 : 2));
      const int nvec = total / EPV;
      for (int v0 = threadIdx.x; v0 < nvec; v0 += kBlock * kBatch) {
        u32x4 x[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
          const int v = v0 + b * kBlock;
          if (v < nvec) x[b] = src[v];
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
          const int v = v0 + b * kBlock;
          if (v < nvec) {
            const int e = v * EPV, r = e / E, c = e - r * E;
#pragma unroll
            for (int t = 0; t < EPV; ++t) {
              uint32_t fb;
              if constexpr (DT == 0) {
                fb = x[b][t];
              } else {
                const uint32_t h = (x[b][t >> 1] >> (16 * (t & 1))) & 0xFFFFu;
                fb = DT == 1 ? __builtin_bit_cast(uint32_t, (float)__builtin_bit_cast(_Float16, (uint16_t)h))
                             : (h << 16);
              }
              lds[r * stride + c + t] = key_of_bits(fb);
            }
          }
        }
      }
    } else {
      for (int e = threadIdx.x; e < total; e += kBlock) lds[(e / E) * stride + e % E] = load_key<DT>(logits, base + e);
    }
  }
  __syncthreads();

  const int r = threadIdx.x / LPR;
  const int q = threadIdx.x % LPR;
  if (r >= nrows) return;  // whole LPR groups leave together (nrows is uniform)

  uint32_t u[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int c = q * V + j;
    u[j] = c < E ? lds[r * stride + c] : 0u;
  }

  uint32_t sel_u[KMAX];
  int sel_i[KMAX];
#pragma unroll
  for (int t = 0; t < KMAX; ++t) {
    if (t < k) {
      uint32_t bu = 0;
      int bi = 0x7FFFFFFF;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const bool gt = u[j] > bu;
        bu = gt ? u[j] : bu;
        bi = gt ? q * V + j : bi;
      }
#pragma unroll
      for (int off = 1; off < LPR; off <<= 1) {
        const uint32_t ou = __shfl_xor(bu, off, LPR);
        const int oi = __shfl_xor(bi, off, LPR);
        const bool take = ou > bu || (ou == bu && oi < bi);
        bu = take ? ou : bu;
        bi = take ? oi : bi;
      }
      sel_u[t] = bu;
      sel_i[t] = bi;
#pragma unroll
      for (int j = 0; j < V; ++j) u[j] = (q * V + j == bi) ? 0u : u[j];
    }
  }

  if (q != 0) return;
  const float v0 = float_of_key(sel_u[0]);
  float e[KMAX];
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < KMAX; ++t) {
    if (t < k) {
      e[t] = expf(float_of_key(sel_u[t]) - v0);
      sum += e[t];
    }
  }
  const int64_t out0 = (row0 + r) * k;
#pragma unroll
  for (int t = 0; t < KMAX; ++t) {
    if (t < k) {
      store_weight<DT>(weights, out0 + t, e[t] / sum);
      indices[out0 + t] = sel_i[t];
    }
  }
}

template <int DT, int V, int LPR, int KMAX>
static tb_status launch(const void* logits, void* weights, int32_t* indices, int64_t M, int E, int k,
                        hipStream_t stream) {
  constexpr int ROWS = kBlock / LPR;
  const size_t lds = (size_t)ROWS * (E + kPad) * sizeof(uint32_t);
  const int64_t blocks = (M + ROWS - 1) / ROWS;
  hipLaunchKernelGGL((gating_kernel<DT, V, LPR, KMAX>), dim3((unsigned)blocks), dim3(kBlock), lds, stream, logits,
                     weights, indices, M, E, k);
  return launch_status("tb_moe_topk_gating");
}

template <int DT, int KMAX>
static tb_status dispatch_shape(const void* logits, void* weights, int32_t* indices, int64_t M, int E, int k,
                                hipStream_t stream) {
  // Lanes per row: enough that V <= 16 values per lane for E <= 64 (fills all
  // four SIMDs of every CU at M = 16k rows) and V = 64 beyond.
  if (E <= 16) return launch<DT, 16, 1, KMAX>(logits, weights, indices, M, E, k, stream);
  if (E <= 32) return launch<DT, 16, 2, KMAX>(logits, weights, indices, M, E, k, stream);
  if (E <= 64) return launch<DT, 16, 4, KMAX>(logits, weights, indices, M, E, k, stream);
  if (E <= 128) return launch<DT, 32, 4, KMAX>(logits, weights, indices, M, E, k, stream);
  if (E <= 256) return launch<DT, 64, 4, KMAX>(logits, weights, indices, M, E, k, stream);
  if (E <= 512) return launch<DT, 64, 8, KMAX>(logits, weights, indices, M, E, k, stream);
  return launch<DT, 64, 16, KMAX>(logits, weights, indices, M, E, k, stream);
}

template <int DT>
static tb_status dispatch_k(const void* logits, void* weights, int32_t* indices, int64_t M, int E, int k,
                            hipStream_t stream) {
  if (k <= 2) return dispatch_shape<DT, 2>(logits, weights, indices, M, E, k, stream);
  if (k <= 8) return dispatch_shape<DT, 8>(logits, weights, indices, M, E, k, stream);
  return dispatch_shape<DT, 32>(logits, weights, indices, M, E, k, stream);
}

}  // namespace tb

extern "C" tb_status tb_moe_topk_gating(const void* logits, void* weights, int32_t* indices, int64_t M, int64_t E,
                                        int64_t k, int dtype, hipStream_t stream) {
  TB_CHECK_ARG(logits && weights && indices, "tb_moe_topk_gating: null pointer");
  TB_CHECK_ARG(M > 0 && E > 0 && E <= 1024, "tb_moe_topk_gating: need M > 0 and 0 < E <= 1024 (M=%lld E=%lld)",
               (long long)M, (long long)E);
  TB_CHECK_ARG(k >= 1 && k <= E && k <= 32, "tb_moe_topk_gating: need 1 <= k <= min(E, 32) (k=%lld E=%lld)",
               (long long)k, (long long)E);
  TB_CHECK_ARG(dtype >= 0 && dtype <= 2, "tb_moe_topk_gating: dtype must be 0 (fp32), 1 (fp16) or 2 (bf16)");
  TB_CHECK_ALIGN(logits, 16, "logits");
  const int e = (int)E, kk = (int)k;
  switch (dtype) {
    case 0: return tb::dispatch_k<0>(logits, weights, indices, M, e, kk, stream);
    case 1: return tb::dispatch_k<1>(logits, weights, indices, M, e, kk, stream);
    default: return tb::dispatch_k<2>(logits, weights, indices, M, e, kk, stream);
  }
}
