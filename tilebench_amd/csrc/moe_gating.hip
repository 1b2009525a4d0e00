// MoE router gating: per row, top-k logits (descending, equal logits -> lowest
// expert index first) and the softmax over those k logits in fp32.
//
// Layout: a row is owned by LPR consecutive lanes (a power of two), lane q
// holding elements q*V .. q*V+V-1 (V = 16) in registers, loaded with 16-byte
// loads: the lanes of a row read it with one contiguous sweep and consecutive
// rows follow, so the logits stream straight from HBM into registers, with no
// LDS staging and no barrier.
//
// Each logit becomes an order-preserving uint32 key, and each (key, index)
// pair one double holding the integer 2^52 + key*1024 + (1023 - index): the
// double order is the selection order (larger key first, then lower index),
// and no two elements of a row are equal, so a compare-exchange is one max
// and one min.  Every lane sorts its V elements (a Batcher network, pruned by
// the compiler to the entries that can be selected).  k rounds follow: the
// LPR lanes take the maximum of their list heads with an xor-butterfly, which
// leaves every lane of the row with the winner, and the lane that held it
// pops its list.  Selection runs on the logits themselves, never on exp()
// values, so rounding in exp cannot create or break ties.  Lane t % LPR
// writes output t (weights and indices of a row land in one coalesced store).
//
// Key map: k(x) = 0x80000000 + |x| bits for x >= 0 and 0x80000000 - |x| bits
// for x < 0, so -0.0 and +0.0 meet at 0x80000000 (they compare equal), and
// every NaN maps to 0xFFFFFFFF (a NaN ranks above +inf, as in torch.topk).
// Real keys are >= k(-inf) = 0x00800000, so 0 marks an absent slot.
#include "tb_common.h"

#include <utility>

namespace tb {

__device__ __forceinline__ uint32_t key_of_bits(uint32_t b) {
  const uint32_t mag = b & 0x7FFFFFFFu;
  const uint32_t neg = (uint32_t)((int32_t)b >> 31);  // all ones when the sign bit is set
  const uint32_t key = 0x80000000u + ((mag ^ neg) - neg);
  return mag > 0x7F800000u ? 0xFFFFFFFFu : key;
}

__device__ __forceinline__ float float_of_key(uint32_t u) {
  const uint32_t b = u >= 0x80000000u ? u - 0x80000000u : 0x80000000u | (0x80000000u - u);
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

// Batcher's odd-even merge sort on N = 2^p inputs as a list of comparators
// (lo, hi): a compare-exchange leaves the larger value at lo, so the network
// sorts descending.  Generated at compile time; fully unrolled, every index is
// a constant and the values stay in registers.
template <int N>
struct SortNet {
  int lo[N * N], hi[N * N];
  int count;
};
template <int N>
constexpr SortNet<N> make_sort_net() {
  SortNet<N> net{};
  net.count = 0;
  for (int p = 1; p < N; p <<= 1)
    for (int d = p; d >= 1; d >>= 1)
      for (int j = d % p; j + d < N; j += 2 * d)
        for (int i = 0; i < d && i + j + d < N; ++i)
          if ((i + j) / (2 * p) == (i + j + d) / (2 * p)) {
            net.lo[net.count] = i + j;
            net.hi[net.count] = i + j + d;
            ++net.count;
          }
  return net;
}

// A lane's elements live in one vector value rather than an array: with an
// array, the compiler turns `pop ? s[i + 1] : s[i]` into a load at a computed
// index and then expands that into a select over every element.
template <int N>
using ElemVec = double __attribute__((ext_vector_type(N)));

template <int N, int LO, int HI>
__device__ __forceinline__ void compare_exchange(ElemVec<N>& s) {
  const double a = s[LO], b = s[HI];
  s[LO] = __builtin_fmax(a, b);
  s[HI] = __builtin_fmin(a, b);
}
// Apply the network to all N elements; each comparator's indices are template
// constants (pack expansion), so no index is computed at run time.
template <int N, size_t... C>
__device__ __forceinline__ void sort_desc(ElemVec<N>& s, std::index_sequence<C...>) {
  constexpr SortNet<N> net = make_sort_net<N>();
  (compare_exchange<N, net.lo[C], net.hi[C]>(s), ...);
}

// An element as one double: the integer 2^52 + (key << 10) + (1023 - index),
// built from its bits (exponent 0x433, no rounding).  Keys are 32-bit and
// indices < 1024, so every value lies in [2^52, 2^53) where doubles are the
// integers, distinct elements of a row give distinct values, and the double
// order is (key descending, then index ascending): ties need no second compare.
// 1023 - index is passed as its lane part (bits the lane's first index fixes)
// and its element part, which share no bit set.
__device__ __forceinline__ double pack_elem(uint32_t key, uint32_t rev_lane, uint32_t rev_elem) {
  const u32x2 b = {(key << 10) | rev_lane | rev_elem, __builtin_amdgcn_alignbit(0x43300000u >> 10, key, 22)};
  return __builtin_bit_cast(double, b);
}
__device__ __forceinline__ uint32_t elem_key(double v) {
  const u32x2 b = __builtin_bit_cast(u32x2, v);
  return (b.y << 22) | (b.x >> 10);
}
__device__ __forceinline__ int elem_index(double v) {
  return 1023 - (int)(__builtin_bit_cast(u32x2, v).x & 1023u);
}

template <int LPR>
__device__ __forceinline__ double xchg_elem(double v, int step) {
  u32x2 b = __builtin_bit_cast(u32x2, v);
  b.x = xchg<LPR>(b.x, step);
  b.y = xchg<LPR>(b.y, step);
  return __builtin_bit_cast(double, b);
}

template <int DT, int V, int LPR, int KMAX>
__global__ void __launch_bounds__(kBlock) gating_kernel(const void* __restrict__ logits, void* __restrict__ weights,
                                                        int32_t* __restrict__ indices, int64_t M, int E, int k) {
  constexpr int ROWS = kBlock / LPR;
  constexpr int ESZ = DT == 0 ? 4 : 2;
  constexpr int L = KMAX < V ? KMAX : V;  // list entries a lane can ever contribute
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

  // The lane's L largest elements, largest first.  Absent elements (past E)
  // have key 0 and rank below every real one; k <= E keeps them unselected.
  ElemVec<V> s;
  {
    // q*V has no bit below V (a power of two), so 1023 - (q*V + j) splits
    // into (1023 - q*V - (V-1)) | (V-1 - j).
    const uint32_t rev_lane = 1023u - (uint32_t)(q * V) - (V - 1);
#pragma unroll
    for (int j = 0; j < V; ++j) s[j] = pack_elem(u[j], rev_lane, (uint32_t)(V - 1 - j));
  }
  if constexpr (L == 2) {
    double m1 = s[0], m2 = 0.0;  // 0.0 lies below every packed value
#pragma unroll
    for (int j = 1; j < V; ++j) {
      const double lo = __builtin_fmin(m1, s[j]);
      m1 = __builtin_fmax(m1, s[j]);
      m2 = __builtin_fmax(m2, lo);
    }
    s[0] = m1;
    s[1] = m2;
  } else if constexpr (V > 1) {
    sort_desc<V>(s, std::make_index_sequence<make_sort_net<V>().count>{});
  }

  // KMAX rounds (straight-line code; those past k are not used): the row's
  // largest remaining element is the maximum of the LPR list heads
  // (xor-butterfly: every lane of the row ends with it), and the lane whose
  // head it is (values are unique in a row) pops its list.  Round t reads
  // only the first KMAX - t entries, so the shifts shrink round by round.
  double sel[KMAX];
#pragma unroll
  for (int t = 0; t < KMAX; ++t) {
    double best = s[0];
#pragma unroll
    for (int step = 0; (1 << step) < LPR; ++step) best = __builtin_fmax(best, xchg_elem<LPR>(best, step));
    sel[t] = best;
    ElemVec<V> next = s;
#pragma unroll
    for (int i = 0; i + 1 < L; ++i) next[i] = s[i + 1];
    next[L - 1] = 0.0;
    s = s[0] == best ? next : s;
  }

  // softmax over the k selected logits in fp32, summed in selection order
  const float v0 = float_of_key(elem_key(sel[0]));
  float e[KMAX];
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < KMAX; ++t) {
    e[t] = 0.f;
    if (t < k) {
      e[t] = expf(float_of_key(elem_key(sel[t])) - v0);
      sum += e[t];
    }
  }
  // Lane q writes outputs q, q + LPR, ...: pick each one's values by selects
  // and divide once per output written.
  const int64_t out0 = r * k;
  constexpr int SLOTS = (KMAX + LPR - 1) / LPR;
#pragma unroll
  for (int m = 0; m < SLOTS; ++m) {
    float em = 0.f;
    double sm = 0.0;
#pragma unroll
    for (int t = m * LPR; t < KMAX && t < (m + 1) * LPR; ++t) {
      const bool mine = t - m * LPR == q;
      em = mine ? e[t] : em;
      sm = mine ? sel[t] : sm;
    }
    const int t = m * LPR + q;
    if (t < k) {
      store_weight<DT>(weights, out0 + t, em / sum);
      indices[out0 + t] = elem_index(sm);
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
