// MoE router gating: per row, top-k logits (descending, equal logits -> lowest
// expert index first) and the softmax over those k logits in fp32.
//
// Layout: a row is owned by LPR consecutive lanes (a power of two), lane q
// holding elements q*V .. q*V+V-1 (V = 16) in registers, loaded with 16-byte
// loads: the lanes of a row read it with one contiguous sweep and consecutive
// rows follow, so the logits stream straight from HBM into registers, with no
// LDS staging and no barrier.  Each logit becomes an order-preserving
// uint32 key.  k selection rounds follow: every lane takes its
// largest remaining key (ascending index order, strict '>', so the lowest index
// wins a tie), the LPR lanes combine (key, index) pairs with xor-shuffles, and
// the owner of the winner clears it.  Selection runs on the logits themselves,
// never on exp() values, so rounding in exp cannot create or break ties.  The
// butterfly leaves every lane of the row with the same k winners, and lane t
// writes output t (weights and indices of a row land in one coalesced store).
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

// Exchange with the partner lane of butterfly step `step` inside a group of
// LPR lanes.  Steps 0-3 (partners within 16 lanes) are DPP moves: quad swaps
// (distance 1 and 2), then the half-row and row mirrors, which pair the two
// 4-lane and the two 8-lane halves; any pairing that joins disjoint halves
// gives the same maximum, and the (key, index) order is total.  Wider steps go
// through the LDS crossbar (__shfl_xor).
template <int LPR>
__device__ __forceinline__ uint32_t xchg(uint32_t v, int step) {
  switch (step) {
    case 0: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    case 1: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    case 2: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false);  // row_half_mirror
    case 3: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false);  // row_mirror
    default: return (uint32_t)__shfl_xor((int)v, 1 << step, LPR);
  }
}

template <int DT, int V, int LPR, int KMAX>
__global__ void __launch_bounds__(kBlock) gating_kernel(const void* __restrict__ logits, void* __restrict__ weights,
                                                        int32_t* __restrict__ indices, int64_t M, int E, int k) {
  constexpr int ROWS = kBlock / LPR;
  constexpr int ESZ = DT == 0 ? 4 : 2;
  const int64_t r = (int64_t)blockIdx.x * ROWS + threadIdx.x / LPR;
  const int q = threadIdx.x % LPR;
  if (r >= M) return;  // whole LPR groups leave together

  // Keys of this lane's elements: one 16-byte load when the chunk lies inside
  // the row and rows are 16-byte multiples (so the load is aligned), else
  // element loads (never past the end of the row).
  uint32_t u[V];
  {
    const int c0 = q * V;
    const char* rowp = reinterpret_cast<const char*>(logits) + (r * E + c0) * ESZ;
    const bool aligned16 = ((E * ESZ) & 15) == 0 && (reinterpret_cast<uintptr_t>(logits) & 15) == 0;
    if (c0 + V <= E && aligned16) {
      constexpr int NV = V * ESZ / 16;
      u32x4 x[NV];
#pragma unroll
      for (int b = 0; b < NV; ++b) x[b] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rowp) + b);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        uint32_t fb;
        if constexpr (DT == 0) {
          fb = x[j / 4][j % 4];
        } else {
          const uint32_t h = (x[j / 8][(j % 8) >> 1] >> (16 * (j & 1))) & 0xFFFFu;
          fb = DT == 1 ? __builtin_bit_cast(uint32_t, (float)__builtin_bit_cast(_Float16, (uint16_t)h)) : (h << 16);
        }
        u[j] = key_of_bits(fb);
      }
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) u[j] = c0 + j < E ? load_key<DT>(logits, r * E + c0 + j) : 0u;
    }
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
      for (int step = 0; (1 << step) < LPR; ++step) {
        const uint32_t ou = xchg<LPR>(bu, step);
        const int oi = (int)xchg<LPR>((uint32_t)bi, step);
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

  // softmax over the k selected logits in fp32, summed in selection order
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
  const int64_t out0 = r * k;
#pragma unroll
  for (int t = 0; t < KMAX; ++t) {
    if (t < k && t % LPR == q) {
      store_weight<DT>(weights, out0 + t, e[t] / sum);
      indices[out0 + t] = sel_i[t];
    }
  }
}

template <int DT, int V, int LPR, int KMAX>
static tb_status launch(const void* logits, void* weights, int32_t* indices, int64_t M, int E, int k,
                        hipStream_t stream) {
  constexpr int ROWS = kBlock / LPR;
  const int64_t blocks = (M + ROWS - 1) / ROWS;
  hipLaunchKernelGGL((gating_kernel<DT, V, LPR, KMAX>), dim3((unsigned)blocks), dim3(kBlock), 0, stream, logits,
                     weights, indices, M, E, k);
  return launch_status("tb_moe_topk_gating");
}

template <int DT, int KMAX>
static tb_status dispatch_shape(const void* logits, void* weights, int32_t* indices, int64_t M, int E, int k,
                                hipStream_t stream) {
  // 16 elements per lane (four 16-byte loads in fp32, two in fp16/bf16) and
  // as many lanes per row as that takes: measured on E in {64, 128, 256}, 16
  // per lane beats 8 (more butterfly work per row) and 32 (fewer wavefronts).
  if (E <= 16) return launch<DT, 16, 1, KMAX>(logits, weights, indices, M, E, k, stream);
  if (E <= 32) return launch<DT, 16, 2, KMAX>(logits, weights, indices, M, E, k, stream);
  if (E <= 64) return launch<DT, 16, 4, KMAX>(logits, weights, indices, M, E, k, stream);
  if (E <= 128) return launch<DT, 16, 8, KMAX>(logits, weights, indices, M, E, k, stream);
  if (E <= 256) return launch<DT, 16, 16, KMAX>(logits, weights, indices, M, E, k, stream);
  if (E <= 512) return launch<DT, 16, 32, KMAX>(logits, weights, indices, M, E, k, stream);
  return launch<DT, 16, 64, KMAX>(logits, weights, indices, M, E, k, stream);
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
