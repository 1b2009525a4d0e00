// MoE router gating: per row, top-k logits (descending, equal logits -> lowest
// expert index first) and the softmax over those k logits in fp32.
//
// Two kernels share the exact selection code below.
//
// filter_kernel (E = 16·V with V in {4, 8, 16} and 2 < k <= 8: the BASELINE
// shapes).  A row is owned by 16 lanes; each lane loads V logits
// with 16-byte loads (8-byte when V·size < 16) laid out so that one load
// instruction of the row's 16 lanes covers 256 contiguous bytes.  Per lane:
//   1. the lane maximum m_q (a med3 chain on the fp32 values) and a flag
//      that is NaN exactly when an element is inf or NaN (a sum of x * 0);
//   2. T = the k-th largest of the 16 lane maxima (a bitonic network across
//      the row's lanes on their signed-int keys, each compare-exchange one
//      max and one min with the partner read by DPP, and a select; for k = 8
//      only the half sorts and a min over the eight largest, eighth_of16_g).
//      The k lanes with the largest maxima hold k distinct elements >= T, so
//      the row's k-th largest element is >= T, and every element the top-k
//      can select is >= T;
//   3. the lane's candidates, elements >= T (float compare: -0 == +0): with
//      V >= 8 a bit mask, with V = 4 the compares themselves and their count;
//   4. the row's candidates are compacted (prefix sum of the lane counts) into
//      an LDS list of exact (key, 1023 - index) pairs (with V >= 8 by a loop
//      over the mask's set bits, each value read back from an LDS copy of the
//      lane's elements; with V = 4 by one masked write per element); with at
//      most 16 of them, lane i takes candidate i and a bitonic network over
//      the 16 lanes sorts them on 32-bit keys that hold the list slot in
//      their low bits, checked against the exact pairs read back by slot
//      (the wavefront sorts the exact pairs when the check fails): lane t
//      ends with the t-th selection.  With 17 to 32, lane i also takes
//      candidate i + 16, both lists are sorted and merged (lane t keeps the
//      larger of list 0's t-th and list 1's (15 - t)-th, a bitonic sequence
//      holding the top 16, sorted by four half-cleaners).
// On random logits a row has about 10 candidates at k = 8; 2.6 % of the
// wavefronts at E = 256 (0.2 % at E = 64) have a row with more than 16, and
// far fewer one with more than 32.  A wavefront any of whose rows has more
// than 32, or holds inf or NaN, runs the exact path below instead (same
// results, more work); with one load per lane (E = 64 in fp32) the lanes
// already hold the exact path's layout, otherwise they read it again.
//
// exact path (every other shape, and the fallback).  A row is owned by LPR
// consecutive lanes (a power of two), lane q holding elements q*V .. q*V+V-1
// in registers.  Each logit becomes an order-preserving uint32 key, and each
// (key, index) pair one double holding the integer 2^52 + key*1024 + (1023 -
// index): the double order is the selection order (larger key first, then
// lower index), and no two elements of a row are equal, so a compare-exchange
// is one max and one min.  Every lane sorts its V elements (a Batcher network,
// pruned by the compiler to the entries that can be selected).  k rounds
// follow: the LPR lanes take the maximum of their list heads with an
// xor-butterfly, which leaves every lane of the row with the winner, and the
// lane that held it pops its list.  Selection runs on the logits themselves,
// never on exp() values, so rounding in exp cannot create or break ties.
// For k <= 2 on fp16/bf16 logits (the reference grid) the selection runs on
// 32-bit (16-bit key, index) values instead (top2_half), falling back to the
// doubles for a wavefront that holds a NaN.
//
// Key map: k(x) = 0x80000000 + |x| bits for x >= 0 and 0x80000000 - |x| bits
// for x < 0, so -0.0 and +0.0 meet at 0x80000000 (they compare equal), and
// every NaN maps to 0xFFFFFFFF (a NaN ranks above +inf, as in torch.topk).
// Real keys are >= k(-inf) = 0x00800000, so 0 marks an absent slot.
//
// The softmax denominator adds the k exponentials in numpy's order for a
// float32 row sum (left to right below 8 terms; 8 strided partial sums joined
// as a tree from 8 on, then the remainder), the order the CPU oracle's
// `e.sum(axis=1, dtype=float32)` uses.
#include "tb_common.h"

#include <utility>

namespace tb {

__device__ __forceinline__ uint32_t key_of_bits(uint32_t b) {
  const uint32_t mag = b & 0x7FFFFFFFu;
  const uint32_t neg = (uint32_t)((int32_t)b >> 31);  // all ones when the sign bit is set
  const uint32_t key = 0x80000000u + ((mag ^ neg) - neg);
  return mag > 0x7F800000u ? 0xFFFFFFFFu : key;
}

// key_of_bits for a finite value (no NaN check): with s the sign mask (0 or
// all ones), b ^ (s | 0x80000000) minus s, i.e. 0x80000000 + |x| bits for
// x >= 0 and 0x80000000 - |x| bits for x < 0 (one bitop3 and one subtract).
__device__ __forceinline__ uint32_t key_of_finite(uint32_t b) {
  const uint32_t sm = (uint32_t)((int32_t)b >> 31);
  return (b ^ (sm | 0x80000000u)) - sm;
}

__device__ __forceinline__ float float_of_key(uint32_t u) {
  const uint32_t b = u >= 0x80000000u ? u - 0x80000000u : 0x80000000u | (0x80000000u - u);
  return __builtin_bit_cast(float, b);
}

// Signed-int order of float bits: for floats a < b, flip(a) < flip(b) as
// int32, with -0.0 just below +0.0; NaN and inf land beyond +-inf's keys.  The
// map is its own inverse.
__device__ __forceinline__ int32_t flip_key(uint32_t b) {
  return (int32_t)(b ^ ((uint32_t)((int32_t)b >> 31) & 0x7FFFFFFFu));
}

// e^x for finite x <= 0: expf's own sequence (x log2 e as a rounded product
// plus its error from an fma and the low part of log2 e, 2^fraction by
// v_exp_f32, scaled by 2^round) without its overflow and underflow tests,
// which only matter outside that range (below about -104 it returns a
// denormal or zero where expf returns zero).
__device__ __forceinline__ float exp_nonpos(float x) {
#pragma clang fp contract(off)
  const float hi = __builtin_bit_cast(float, 0x3FB8AA3Bu);  // log2(e) rounded to fp32
  const float lo = __builtin_bit_cast(float, 0x32A5705Fu);  // log2(e) - hi
  const float ph = x * hi;
  const float pl = __builtin_fmaf(x, lo, __builtin_fmaf(x, hi, -ph));
  const float r = __builtin_rintf(ph);
  return __builtin_ldexpf(__builtin_amdgcn_exp2f((ph - r) + pl), (int)r);
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays a quiet NaN).
__device__ __forceinline__ uint16_t bf16_rne(float f) {
  const uint32_t b = __builtin_bit_cast(uint32_t, f);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x40u);
  return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

// fp32 bits of element `j` of a logits word (fp32: the word; fp16/bf16: half
// j & 1 of the word).
template <int DT>
__device__ __forceinline__ uint32_t f32_bits(uint32_t word, int half) {
  if constexpr (DT == 0) {
    return word;
  } else {
    const uint32_t h = half ? word >> 16 : word & 0xFFFFu;
    if constexpr (DT == 1) return __builtin_bit_cast(uint32_t, (float)__builtin_bit_cast(_Float16, (uint16_t)h));
    return h << 16;
  }
}

template <int DT>
__device__ __forceinline__ uint32_t load_key(const void* base, int64_t i) {
  if constexpr (DT == 0) {
    return key_of_bits(reinterpret_cast<const uint32_t*>(base)[i]);
  } else {
    const uint16_t h = reinterpret_cast<const uint16_t*>(base)[i];
    return key_of_bits(f32_bits<DT>(h, 0));
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

// numpy's float32 sum of e[0 .. n-1] (n <= N): a left-to-right loop below 8
// terms; from 8 on, eight partial sums r[j] = e[j] + e[j+8] + ... over the
// whole blocks of 8, joined as ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), then the
// remaining n % 8 terms left to right.
template <int N>
__device__ __forceinline__ float np_sum(const float (&e)[N], int n) {
  float s = e[0];
  if (N < 8 || n < 8) {
#pragma unroll
    for (int t = 1; t < (N < 8 ? N : 8); ++t)
      if (t < n) s += e[t];
    return s;
  }
  if constexpr (N >= 8) {
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = e[j];
    const int whole = n - n % 8;
#pragma unroll
    for (int i = 8; i + 8 <= N; i += 8)
      if (i < whole) {
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] += e[i + j];
      }
    s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
#pragma unroll
    for (int t = 8; t < N; ++t)
      if (t >= whole && t < n) s += e[t];
  }
  return s;
}

constexpr int kBlock = 256;
// Threads per filter-kernel block: one wavefront (measured 1-4 % faster than
// blocks of 128 or 256 threads).
constexpr int kFilterBlock = 64;

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

// Exact selection: lane q of the row's LPR lanes holds the keys of elements
// q*V .. q*V+V-1 in u; every lane of the row returns the row's KMAX largest
// elements (packed as above), largest first.
template <int V, int LPR, int KMAX>
__device__ __forceinline__ void exact_select(const uint32_t (&u)[V], int q, double (&sel)[KMAX]) {
  constexpr int L = KMAX < V ? KMAX : V;  // list entries a lane can ever contribute

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
  // head it is (values are unique in a row) pops its list.
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
}

// Softmax over the row's k selections (every lane of the row holds all of
// them) and the stores: lane q writes outputs q, q + LPR, ...
template <int DT, int LPR, int KMAX>
__device__ __forceinline__ void write_selected(const double (&sel)[KMAX], int64_t r, int q, int k,
                                               void* __restrict__ weights, int32_t* __restrict__ indices) {
  const float v0 = float_of_key(elem_key(sel[0]));
  float e[KMAX];
#pragma unroll
  for (int t = 0; t < KMAX; ++t) e[t] = t < k ? expf(float_of_key(elem_key(sel[t])) - v0) : 0.f;
  e[0] = (v0 - v0) + 1.f;  // expf(v0 - v0): 1, or NaN for an infinite v0 (inf - inf)
  const float sum = np_sum<KMAX>(e, k);
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

// k <= 2 on fp16 / bf16 logits without NaN: the selection in 32-bit integers.
// A half's order key is 16 bits wide (the 32-bit key of its exact fp32 value,
// shifted right by 16, for the same order and ties), so an element is one
// uint32, key16 << 16 | (1023 - index), and no two elements of a row are
// equal.  The keys of two halves come from packed 16-bit operations on the
// loaded word (finite map: h ^ (s | 0x8000) - s, s the half's sign mask);
// inf needs no special case, and a wavefront holding a NaN (whose key is the
// largest) returns false for the general path.  Within a lane the low bits
// hold 15 - j (element j of the lane's 16); the lane's part of 1023 - index,
// 1008 - 16q, is ORed in after the lane's top two are found (pairs sorted,
// then merged into the running pair).  The rows' top two follow from the
// same merge across the LPR lanes (butterfly), and the outputs from the
// general path's formulas: expf(v_t - v_0), the sum left to right, the
// quotient rounded once to the logits dtype.
template <int DT, int LPR>
__device__ __forceinline__ bool top2_half(const void* __restrict__ logits, void* __restrict__ weights,
                                          int32_t* __restrict__ indices, int64_t r, int q, int E, int k) {
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  constexpr int V = 16;
  constexpr uint32_t NAN_MAG = DT == 1 ? 0x7C00u : 0x7F80u;  // |h| above this is NaN
  const int c0 = q * V;
  uint32_t m1 = 0, m2 = 0;  // the lane's top two, m1 > m2 (0: none)
  bool nan = false;
  auto put2 = [&](uint32_t a, uint32_t b) {  // merge two elements into (m1, m2)
    const uint32_t hi = a > b ? a : b, lo = a > b ? b : a;
    const uint32_t x = m1 < hi ? m1 : hi;
    m1 = m1 > hi ? m1 : hi;
    m2 = m2 > lo ? m2 : lo;
    m2 = m2 > x ? m2 : x;
  };
  const bool aligned16 = ((E * 2) & 15) == 0 && (reinterpret_cast<uintptr_t>(logits) & 15) == 0;
  if (c0 + V <= E && aligned16) {
    const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(logits) + r * E + c0);
    const u32x4 x0 = __builtin_nontemporal_load(p), x1 = __builtin_nontemporal_load(p + 1);
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[i] = x0[i];
      w[4 + i] = x1[i];
    }
    u16x2 mag = {0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const u16x2 mi = __builtin_bit_cast(u16x2, w[i] & 0x7FFF7FFFu);
      mag = __builtin_elementwise_max(mag, mi);
      const uint32_t sm = __builtin_bit_cast(uint32_t, __builtin_bit_cast(s16x2, w[i]) >> (short)15);
      const uint32_t key = __builtin_bit_cast(
          uint32_t, __builtin_bit_cast(u16x2, w[i] ^ (sm | 0x80008000u)) - __builtin_bit_cast(u16x2, sm));
      // element 2i in the low half, 2i + 1 in the high half
      put2((key << 16) | (uint32_t)(15 - 2 * i), (key & 0xFFFF0000u) | (uint32_t)(14 - 2 * i));
    }
    nan = mag.x > NAN_MAG || mag.y > NAN_MAG;
  } else {
    const uint16_t* rowp = reinterpret_cast<const uint16_t*>(logits) + r * E;
#pragma unroll
    for (int j = 0; j < V; j += 2) {
      uint32_t c[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int e = c0 + j + h;
        const uint32_t b = e < E ? rowp[e] : 0u;
        const uint32_t sm = (b & 0x8000u) ? 0xFFFFu : 0u;
        nan = nan || (e < E && (b & 0x7FFFu) > NAN_MAG);
        c[h] = e < E ? ((((b ^ (sm | 0x8000u)) - sm) & 0xFFFFu) << 16) | (uint32_t)(15 - j - h) : 0u;
      }
      put2(c[0], c[1]);
    }
  }
  if (__builtin_amdgcn_ballot_w64(nan) != 0) return false;
  const uint32_t lane_rev = 1008u - 16u * (uint32_t)q;  // 1023 - (c0 + j) = lane_rev | (15 - j)
  m1 = m1 != 0 ? m1 | lane_rev : 0u;
  m2 = m2 != 0 ? m2 | lane_rev : 0u;
#pragma unroll
  for (int step = 0; (1 << step) < LPR; ++step) {
    const uint32_t p1 = xchg<LPR>(m1, step), p2 = xchg<LPR>(m2, step);
    const uint32_t x = m1 < p1 ? m1 : p1;
    m1 = m1 > p1 ? m1 : p1;
    m2 = m2 > p2 ? m2 : p2;
    m2 = m2 > x ? m2 : x;
  }
  // fp32 values of the two selections from their 16-bit keys
  auto value = [](uint32_t m) {
    const uint32_t kk = m >> 16;
    const uint32_t h = kk >= 0x8000u ? kk - 0x8000u : 0x8000u | (0x8000u - kk);
    if constexpr (DT == 1) return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    return __builtin_bit_cast(float, h << 16);
  };
  const float v0 = value(m1);
  // expf(v0 - v0): 1 for finite v0, NaN for an infinite one (inf - inf)
  const float e0 = (v0 - v0) + 1.f, e1 = k > 1 ? expf(value(m2) - v0) : 0.f;
  const float sum = k > 1 ? e0 + e1 : e0;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (t < k && (LPR == 1 ? q == 0 : q == t)) {
      const uint32_t m = t == 0 ? m1 : m2;
      store_weight<DT>(weights, r * k + t, (t == 0 ? e0 : e1) / sum);
      indices[r * k + t] = 1023 - (int)(m & 0xFFFFu);
    }
  }
  return true;
}

template <int DT, int V, int LPR, int KMAX>
__global__ void __launch_bounds__(kBlock) gating_kernel(const void* __restrict__ logits, void* __restrict__ weights,
                                                        int32_t* __restrict__ indices, int64_t M, int E, int k) {
  constexpr int ROWS = kBlock / LPR;
  constexpr int ESZ = DT == 0 ? 4 : 2;
  const int64_t r = (int64_t)blockIdx.x * ROWS + threadIdx.x / LPR;
  const int q = threadIdx.x % LPR;
  if (r >= M) return;  // whole LPR groups leave together
  if constexpr (KMAX == 2 && DT != 0 && V == 16) {
    if (top2_half<DT, LPR>(logits, weights, indices, r, q, E, k)) return;
  }

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
        const int w = j * ESZ / 4;
        u[j] = key_of_bits(f32_bits<DT>(x[w / 4][w % 4], j & 1));
      }
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) u[j] = c0 + j < E ? load_key<DT>(logits, r * E + c0 + j) : 0u;
    }
  }
  double sel[KMAX];
  exact_select<V, LPR, KMAX>(u, q, sel);
  write_selected<DT, LPR, KMAX>(sel, r, q, k, weights, indices);
}

// ------------------------------------------------------------------ filter kernel

// Value of the partner lane in a 16-lane sorting stage (p = lane & 15).
// KIND: 0 = p ^ 1, 1 = p ^ 2 (quad permutes), 2 = p ^ 4 (ds_swizzle, bit mode:
// and 0x1F, xor 4), 3 = p ^ 3 (quad reverse), 4 = p ^ 7 (row_half_mirror),
// 5 = p ^ 15 (row_mirror).  The kernel is VALU-bound, and the swizzle runs on
// the LDS unit where two DPP row shifts and a select would take VALU slots.
template <int KIND>
__device__ __forceinline__ uint32_t partner16(uint32_t v) {
  if constexpr (KIND == 0) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
  if constexpr (KIND == 1) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
  if constexpr (KIND == 2) return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x101F);
  if constexpr (KIND == 3) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x1B, 0xF, 0xF, false);
  if constexpr (KIND == 4) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false);
  if constexpr (KIND == 5) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false);
  if constexpr (KIND == 6) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false);  // row_ror:8
}

// Partner at distance 4 (lane p ^ 4) from two DPP row rotations, which stay
// off the LDS crossbar: row_ror:n hands lane p the value of lane (p - n) % 16,
// so lanes with bit 2 set read through row_ror:4, the others row_ror:12.
__device__ __forceinline__ uint32_t xor4_16(uint32_t v, int p) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xF, 0xF, false);  // row_ror:4: p - 4
  const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x12C, 0xF, 0xF, false);  // row_ror:12: p + 4
  return (p & 4) ? lo : hi;
}
template <int KIND>
__device__ __forceinline__ uint32_t partner16p(uint32_t v, int p) {
  if constexpr (KIND == 2) return xor4_16(v, p);
  return partner16<KIND>(v);
}
template <int KIND, int BIT>
__device__ __forceinline__ int32_t cx_i32(int32_t v, int p) {
  const int32_t w = (int32_t)partner16p<KIND>((uint32_t)v, p);
  return (p & BIT) ? (v < w ? v : w) : (v > w ? v : w);
}
template <int KIND, int BIT>
__device__ __forceinline__ uint64_t cx_u64(uint64_t v, int p) {
  const u32x2 b = __builtin_bit_cast(u32x2, v);
  const u32x2 o = {partner16p<KIND>(b.x, p), partner16p<KIND>(b.y, p)};
  const uint64_t w = __builtin_bit_cast(uint64_t, o);
  return ((v > w) == ((p & BIT) == 0)) ? v : w;
}
// Lane n of the caller's 16-lane row, broadcast to the row (DPP row_newbcast).
template <int N>
__device__ __forceinline__ uint32_t row_bcast(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x150 + N, 0xF, 0xF, false);
}
template <int N>
__device__ __forceinline__ float row_bcast_f(float v) {
  return __builtin_bit_cast(float, row_bcast<N>(__builtin_bit_cast(uint32_t, v)));
}
// e[t] = lane t's x, for every t of the sequence
template <int... T, size_t N>
__device__ __forceinline__ void bcast_all(float x, float (&e)[N], std::integer_sequence<int, T...>) {
  ((e[T] = row_bcast_f<T>(x)), ...);
}
// Lane n (0 <= n < 8, wave-uniform) of the row, broadcast to the row.
__device__ __forceinline__ uint32_t row_bcast_lt8(uint32_t v, int n) {
  switch (n) {
    case 0: return row_bcast<0>(v);
    case 1: return row_bcast<1>(v);
    case 2: return row_bcast<2>(v);
    case 3: return row_bcast<3>(v);
    case 4: return row_bcast<4>(v);
    case 5: return row_bcast<5>(v);
    case 6: return row_bcast<6>(v);
    default: return row_bcast<7>(v);
  }
}

// Descending sort of one value per lane across the 16 lanes of a row (p = lane
// & 15 ends holding the p-th largest).  Bitonic sort in its mirror form: the
// first stage of each merge of two sorted blocks compares lane i with its
// mirror in the merged block, the later stages are half-cleaners at distances
// 4, 2, 1; the lower lane of each pair keeps the larger value.
__device__ __forceinline__ int32_t sort16_desc(int32_t v, int p) {
  v = cx_i32<0, 1>(v, p);
  v = cx_i32<3, 2>(v, p);
  v = cx_i32<0, 1>(v, p);
  v = cx_i32<4, 4>(v, p);
  v = cx_i32<1, 2>(v, p);
  v = cx_i32<0, 1>(v, p);
  v = cx_i32<5, 8>(v, p);
  v = cx_i32<2, 4>(v, p);
  v = cx_i32<1, 2>(v, p);
  return cx_i32<0, 1>(v, p);
}
__device__ __forceinline__ uint64_t sort16_desc(uint64_t v, int p) {
  v = cx_u64<0, 1>(v, p);
  v = cx_u64<3, 2>(v, p);
  v = cx_u64<0, 1>(v, p);
  v = cx_u64<4, 4>(v, p);
  v = cx_u64<1, 2>(v, p);
  v = cx_u64<0, 1>(v, p);
  v = cx_u64<5, 8>(v, p);
  v = cx_u64<2, 4>(v, p);
  v = cx_u64<1, 2>(v, p);
  return cx_u64<0, 1>(v, p);
}

// Partner value for a compare-exchange whose move the compiler folds into the
// min / max that use it (v_max_i32_dpp): bound_ctrl with a zero old value.
// Every pattern used here is a permutation of the 16-lane row, so no lane
// reads outside it.
template <int CTRL>
__device__ __forceinline__ int32_t dpp_i32(int32_t v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, dpp_i32<CTRL>(__builtin_bit_cast(int32_t, v)));
}
// Compare-exchange of one sorting stage: the lane keeps the larger value
// unless (p & BIT), CTRL naming the partner (p ^ 1, p ^ 3, p ^ 7, p ^ 15 or
// p ^ 2).
template <int CTRL, int BIT>
__device__ __forceinline__ int32_t cxf_i32(int32_t v, int p) {
  const int32_t hi = max(v, dpp_i32<CTRL>(v)), lo = min(v, dpp_i32<CTRL>(v));
  return (p & BIT) ? lo : hi;
}
// The distance-4 stage (partner p ^ 4, BIT = 4): lanes with bit 2 set keep
// the minimum with lane p - 4 (row_ror:4), the others the maximum with lane
// p + 4 (row_ror:12).
__device__ __forceinline__ int32_t cxf4_i32(int32_t v, int p) {
  const int32_t lo = min(v, dpp_i32<0x124>(v)), hi = max(v, dpp_i32<0x12C>(v));
  return (p & 4) ? lo : hi;
}
// sort16_desc on G independent values per lane (rows of a lane group), stage
// by stage, so the rows' dependent chains interleave.
template <int G>
__device__ __forceinline__ void sort16_desc_g(int32_t (&v)[G], int p) {
#define TB_STAGE(expr)            \
  _Pragma("unroll") for (int g = 0; g < G; ++g) { \
    const int32_t x = v[g];       \
    v[g] = expr;                  \
  }
  TB_STAGE((cxf_i32<0xB1, 1>(x, p)))
  TB_STAGE((cxf_i32<0x1B, 2>(x, p)))
  TB_STAGE((cxf_i32<0xB1, 1>(x, p)))
  TB_STAGE((cxf_i32<0x141, 4>(x, p)))
  TB_STAGE((cxf_i32<0x4E, 2>(x, p)))
  TB_STAGE((cxf_i32<0xB1, 1>(x, p)))
  TB_STAGE((cxf_i32<0x140, 8>(x, p)))
  TB_STAGE((cxf4_i32(x, p)))
  TB_STAGE((cxf_i32<0x4E, 2>(x, p)))
  TB_STAGE((cxf_i32<0xB1, 1>(x, p)))
}

// The 8th largest of the 16 values of a row, in every lane of the row, for G
// rows per lane group.  The first six stages of sort16_desc sort each 8-lane
// half descending (a, b); the larger of lane i and its mirror 15 - i,
// max(a[i], b[7 - i]), leaves the row's eight largest values in each half (the
// bitonic merge's first step), and their minimum is reduced over the half:
// 22 VALU operations per row against 31 for the full sort and a broadcast.
template <int G>
__device__ __forceinline__ void eighth_of16_g(int32_t (&v)[G], int p) {
  TB_STAGE((cxf_i32<0xB1, 1>(x, p)))
  TB_STAGE((cxf_i32<0x1B, 2>(x, p)))
  TB_STAGE((cxf_i32<0xB1, 1>(x, p)))
  TB_STAGE((cxf_i32<0x141, 4>(x, p)))
  TB_STAGE((cxf_i32<0x4E, 2>(x, p)))
  TB_STAGE((cxf_i32<0xB1, 1>(x, p)))
  TB_STAGE((max(x, dpp_i32<0x140>(x))))  // row_mirror: lane 15 - i
  TB_STAGE((min(x, dpp_i32<0xB1>(x))))   // lane i ^ 1
  TB_STAGE((min(x, dpp_i32<0x4E>(x))))   // lane i ^ 2
  TB_STAGE((min(x, dpp_i32<0x141>(x))))  // row_half_mirror: the other quad of the half
#undef TB_STAGE
}

// Lane n (0 <= n < 16, a run-time value) of the caller's 16-lane row, through
// the LDS crossbar (ds_bpermute).
__device__ __forceinline__ int32_t row_lane(int32_t v, int n) {
  const int src = (int)(threadIdx.x & 48u) + n;
  return __builtin_amdgcn_ds_bpermute(src << 2, v);
}

// Geometry of the filter kernel for E = 16·V elements of ESZ bytes.
template <int DT, int V>
struct FilterShape {
  static constexpr int LPR = 16;                          // lanes per row
  static constexpr int E = LPR * V;
  static constexpr int ESZ = DT == 0 ? 4 : 2;
  static constexpr int ROWB = E * ESZ;                    // bytes per row
  static constexpr int CB = V * ESZ < 16 ? V * ESZ : 16;  // bytes per load
  static constexpr int NC = V * ESZ / CB;                 // loads per lane
  static constexpr int EPC = CB / ESZ;                    // elements per load
  static constexpr int CW = CB / 4;                       // words per load
  static constexpr int ROWS = kFilterBlock / LPR;         // rows of a row group
  static constexpr bool STAGED = V >= 8;                  // candidates gathered from an LDS copy
  static constexpr int SSTRIDE = V + 4;                   // words per lane of that copy (16-byte multiple)
  static_assert(CB == 8 || CB == 16, "filter_kernel: 8- or 16-byte loads");
};

// A block owns G row groups of ROWS consecutive rows: group g holds rows
// G*ROWS*blockIdx.x + g*ROWS .. +ROWS-1, one row per 16 lanes, so each lane
// group works on G rows at once, every step issued for all of them together
// (their dependent chains interleave, and the grid has G times fewer
// wavefronts to dispatch).  Every load goes through a buffer resource over the
// block's rows: rows past M read zeros, move no data and are not stored.
template <int DT, int V, int KMAX, int G, bool KFIX>
__global__ void __launch_bounds__(kFilterBlock) filter_kernel(const void* __restrict__ logits, void* __restrict__ weights,
                                                        int32_t* __restrict__ indices, int64_t M, int k) {
  if constexpr (KFIX) k = KMAX;  // k == KMAX known at compile time (the BASELINE k = 8)
  using S = FilterShape<DT, V>;
  constexpr int LPR = S::LPR, ESZ = S::ESZ, ROWB = S::ROWB, CB = S::CB, NC = S::NC, EPC = S::EPC, CW = S::CW,
                ROWS = S::ROWS;
  constexpr int NT = 2;  // nontemporal: every logit is read once
  constexpr int DUMMY = 2 * LPR;  // list entry taking the writes of lanes with nothing to write

  __shared__ uint64_t cand[G][ROWS][2 * LPR + 1];
  __shared__ uint32_t staged[S::STAGED ? G * kFilterBlock * S::SSTRIDE : 1];

  const int slot = threadIdx.x / LPR;
  const int q = threadIdx.x % LPR;
  const int64_t r0 = (int64_t)blockIdx.x * (ROWS * G);
  const int64_t here = M - r0 < (int64_t)(ROWS * G) ? M - r0 : (int64_t)(ROWS * G);  // rows of this block
  const buf_rsrc_t rl = buf_rsrc(reinterpret_cast<const char*>(logits) + r0 * ROWB, (uint32_t)(here * ROWB));

  // Load c of lane q covers row elements c*16*EPC + q*EPC + (0 .. EPC-1), so
  // one load instruction of a row's lanes reads 16*CB contiguous bytes.
  uint32_t w[G][NC * CW];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int row = g * ROWS + slot;
    const uint32_t base = row < here ? (uint32_t)(row * ROWB + q * CB) : BUF_OOB;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if constexpr (CB == 16) {
        const u32x4 x = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rl, base, c * LPR * CB, NT));
#pragma unroll
        for (int i = 0; i < 4; ++i) w[g][c * 4 + i] = x[i];
      } else {
        const u32x2 x = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rl, base, c * LPR * CB, NT));
#pragma unroll
        for (int i = 0; i < 2; ++i) w[g][c * 2 + i] = x[i];
      }
    }
  }
  bool live[G];
#pragma unroll
  for (int g = 0; g < G; ++g) live[g] = g * ROWS + slot < here;

  // fp32 values of the lane's elements, j = c*EPC + i; the lane maximum
  // (med3 with +inf is the larger of two finite values) and a flag that is NaN
  // exactly when an element is not finite (x * 0 is NaN for inf and NaN).
  float f[G][V];
  int32_t kmax[G];
  bool finite = true;
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int j = 0; j < V; ++j) f[g][j] = __builtin_bit_cast(float, f32_bits<DT>(w[g][j * ESZ / 4], j & 1));
    float mx = f[g][0], nf0 = 0.f, nf1 = 0.f;
#pragma unroll
    for (int j = 1; j < V; ++j) mx = __builtin_amdgcn_fmed3f(mx, f[g][j], __builtin_inff());
#pragma unroll
    for (int j = 0; j < V; j += 2) {
      nf0 = __builtin_fmaf(f[g][j], 0.f, nf0);
      if (j + 1 < V) nf1 = __builtin_fmaf(f[g][j + 1], 0.f, nf1);
    }
    finite = finite && (nf0 + nf1 == 0.f);
    kmax[g] = flip_key(__builtin_bit_cast(uint32_t, mx));
  }
  if constexpr (S::STAGED) {
    // the lane's elements, for the candidate gather below
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < V; j += 4)
        *reinterpret_cast<u32x4*>(&staged[(g * kFilterBlock + threadIdx.x) * S::SSTRIDE + j]) =
            __builtin_bit_cast(u32x4, f32x4{f[g][j], f[g][j + 1], f[g][j + 2], f[g][j + 3]});
  }

  // T = the k-th largest lane maximum of the row (k <= KMAX = 8): the k lanes
  // above it hold k elements >= T, so every element the top-k can select is >= T.
  constexpr bool EIGHTH = KFIX && KMAX == 8;
  if constexpr (EIGHTH)
    eighth_of16_g<G>(kmax, q);
  else
    sort16_desc_g<G>(kmax, q);
  float T[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int32_t tk = EIGHTH ? kmax[g]
                       : KFIX ? (int32_t)row_bcast<KMAX - 1>((uint32_t)kmax[g])
                              : row_lane(kmax[g], k - 1);
    T[g] = __builtin_bit_cast(float, (uint32_t)flip_key((uint32_t)tk));
  }

  // candidate mask (bit j for element j), counts and their inclusive prefix
  // across the row's 16 lanes
  // Below eight elements per lane the per-element compares are kept as they
  // are (lane masks the gather branches on) and the count is their running sum.
  constexpr bool FLAGS = !S::STAGED;
  uint32_t mask[G];
  bool ge[G][FLAGS ? V : 1];
  int cnt[G], incl[G], total[G];
  bool fast = finite;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if constexpr (FLAGS) {
      int c = 0;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        ge[g][j] = f[g][j] >= T[g];
        c += (int)ge[g][j];
      }
      cnt[g] = c;
    } else {
      uint32_t m = 0;
#pragma unroll
      for (int j = V - 1; j >= 0; --j) m = m + m + (uint32_t)(f[g][j] >= T[g]);
      mask[g] = live[g] ? m : 0u;  // rows past M (zeros) have no candidates: nothing is written for them
      cnt[g] = __builtin_popcount(m);
    }
    int x = cnt[g];
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);  // row_shr:8
    incl[g] = x;
    total[g] = (int)row_bcast<LPR - 1>((uint32_t)x);
    fast = fast && (!live[g] || total[g] <= 2 * LPR);
  }

  if (__builtin_amdgcn_ballot_w64(!fast) == 0) {
    // Each candidate goes to the row's LDS list as the exact (key, 1023 - index)
    // pair, at its slot among the row's: the lane's base plus its candidates
    // before it.
    if constexpr (S::STAGED) {
      // a loop over the set bits of the masks (about one candidate per lane),
      // each candidate's value read back from the lane's LDS copy; a lane
      // with nothing left in a row writes to the row's spare entry
      uint32_t m[G];
      int dst[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        m[g] = mask[g];
        dst[g] = incl[g] - cnt[g];
      }
      uint32_t any = 0;
#pragma unroll
      for (int g = 0; g < G; ++g) any |= m[g];
      while (any != 0) {
        any = 0;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const bool has = m[g] != 0;
          const int j = has ? __builtin_ctz(m[g]) : 0;
          m[g] &= m[g] - 1u;
          const uint32_t fj = staged[(g * kFilterBlock + threadIdx.x) * S::SSTRIDE + j];
          const int idx = (j / EPC) * (LPR * EPC) + q * EPC + (j % EPC);
          cand[g][slot][has ? dst[g] : DUMMY] = ((uint64_t)key_of_finite(fj) << 32) | (uint32_t)(1023 - idx);
          dst[g] += has;
          any |= m[g];
        }
      }
    } else {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        // rows past M (zeros) have no candidates: nothing is written for them
        int dst = incl[g] - cnt[g];
#pragma unroll
        for (int j = 0; j < V; ++j) {
          if (live[g] && ge[g][j]) {
            const int idx = (j / EPC) * (LPR * EPC) + q * EPC + (j % EPC);
            cand[g][slot][dst] =
                ((uint64_t)key_of_finite(__builtin_bit_cast(uint32_t, f[g][j])) << 32) | (uint32_t)(1023 - idx);
          }
          dst += (int)ge[g][j];
        }
      }
    }
    // The lists are read by other lanes of this wavefront only (each
    // wavefront owns its rows' LDS), so a wavefront-scope fence orders the
    // accesses.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // lane q takes candidate q; 0 marks no candidate
    uint64_t v[G];
    bool big = false;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      v[g] = q < total[g] ? cand[g][slot][q] : 0;
      big = big || (live[g] && total[g] > LPR);
    }
    if (__builtin_amdgcn_ballot_w64(big) == 0) {
      // Sorted on 32-bit keys: a candidate's order key with its low five bits
      // replaced by 31 - its list slot (sign flipped for the signed sort;
      // valid order keys exceed 2^23, so an empty lane's INT32_MIN sorts last).
      // Lane t then reads its exact (key, 1023 - index) pair back from the
      // list by that slot.  The short keys order the candidates exactly unless
      // two of them differ only in the dropped bits, which the check below
      // finds as an adjacent pair out of order; the wavefront then sorts the
      // exact pairs.
      int32_t c[G];
#pragma unroll
      for (int g = 0; g < G; ++g)
        c[g] = q < total[g] ? (int32_t)((((uint32_t)(v[g] >> 32) & ~31u) | (uint32_t)(31 - q)) ^ 0x80000000u)
                            : INT32_MIN;
      sort16_desc_g<G>(c, q);
      bool bad = false;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        v[g] = q < total[g] ? cand[g][slot][31 - (c[g] & 31)] : 0;
        const u32x2 b = __builtin_bit_cast(u32x2, v[g]);
        const uint64_t next = __builtin_bit_cast(
            uint64_t, u32x2{(uint32_t)__builtin_amdgcn_update_dpp(0, (int)b.x, 0x101, 0xF, 0xF, true),
                            (uint32_t)__builtin_amdgcn_update_dpp(0, (int)b.y, 0x101, 0xF, 0xF, true)});  // row_shl:1
        bad = bad || (q < total[g] && v[g] <= next);
      }
      if (__builtin_amdgcn_ballot_w64(bad) != 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) v[g] = sort16_desc(v[g], q);
      }
    } else {
      // a row of this wavefront has 17..32 candidates: lane q also takes
      // candidate q + 16, both lists are sorted, and lane t keeps the larger
      // of v[t] and v1[15 - t]; those 16 are the top 16 of the union as a
      // bitonic sequence, which the half-cleaners at distances 8, 4, 2, 1 sort
#pragma unroll
      for (int g = 0; g < G; ++g) {
        uint64_t v1 = q + LPR < total[g] ? cand[g][slot][q + LPR] : 0;
        v[g] = sort16_desc(v[g], q);
        v1 = sort16_desc(v1, q);
        const u32x2 b = __builtin_bit_cast(u32x2, v1);
        const uint64_t mm = __builtin_bit_cast(uint64_t, u32x2{partner16<5>(b.x), partner16<5>(b.y)});
        v[g] = v[g] > mm ? v[g] : mm;
        v[g] = cx_u64<6, 8>(v[g], q);
        v[g] = cx_u64<2, 4>(v[g], q);
        v[g] = cx_u64<1, 2>(v[g], q);
        v[g] = cx_u64<0, 1>(v[g], q);
      }
    }

    // lane t < k holds selection t of its row
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float val = float_of_key((uint32_t)(v[g] >> 32));
      const float v0 = row_bcast_f<0>(val);
      const float et = q < k ? exp_nonpos(val - v0) : 0.f;  // val <= v0, the row maximum
      float sum;
      if constexpr (EIGHTH) {
        // np_sum's order for 8 terms, ((e0 + e1) + (e2 + e3)) + ((e4 + e5) +
        // (e6 + e7)), as a tree over lanes 0..7, each level adding the partial
        // sum of the partner lane (p ^ 1, p ^ 2, then the other quad of the
        // half): addition commutes, so every lane of the half ends with the
        // same bits.
        sum = et;
        sum += dpp_f32<0xB1>(sum);
        sum += dpp_f32<0x4E>(sum);
        sum += dpp_f32<0x141>(sum);
      } else {
        float e[KMAX];
        bcast_all(et, e, std::make_integer_sequence<int, KMAX>{});
        sum = np_sum<KMAX>(e, k);
      }
      const int64_t r = r0 + g * ROWS + slot;
      if (live[g] && q < k) {
        store_weight<DT>(weights, r * k + q, et / sum);
        indices[r * k + q] = 1023 - (int)(uint32_t)v[g];
      }
    }
  } else {
    // exact path for every row of the wavefront: lane q takes elements
    // q*V .. q*V+V-1.  With one load per lane it already holds them;
    // otherwise it reads them again (this path is rare).  Unrolled: a
    // run-time row index into f would move f out of registers.
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (!live[g]) continue;
      const int64_t r = r0 + g * ROWS + slot;
      uint32_t u[V];
      if constexpr (NC == 1) {
#pragma unroll
        for (int j = 0; j < V; ++j) u[j] = key_of_bits(__builtin_bit_cast(uint32_t, f[g][j]));
      } else {
        const uint32_t* rw = reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(logits) + r * ROWB) +
                             q * V * ESZ / 4;
        uint32_t x[V * ESZ / 4];
#pragma unroll
        for (int c = 0; c < V * ESZ / 16; ++c) {
          const u32x4 t = *reinterpret_cast<const u32x4*>(rw + 4 * c);
#pragma unroll
          for (int i = 0; i < 4; ++i) x[4 * c + i] = t[i];
        }
#pragma unroll
        for (int j = 0; j < V; ++j) u[j] = key_of_bits(f32_bits<DT>(x[j * ESZ / 4], j & 1));
      }
      double sel[KMAX];
      exact_select<V, LPR, KMAX>(u, q, sel);
      write_selected<DT, LPR, KMAX>(sel, r, q, k, weights, indices);
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

template <int DT, int V, int KMAX>
static tb_status launch_filter(const void* logits, void* weights, int32_t* indices, int64_t M, int k,
                               hipStream_t stream) {
  // One row per lane group: two or four rows per lane group (half or a
  // quarter of the wavefronts, each row's steps interleaved with the others')
  // measured 20-60 % slower, the wavefronts hiding each other's latencies
  // better than a wavefront's rows do.
  constexpr int G = 1;
  constexpr int ROWS = kFilterBlock / 16;
  const int64_t blocks = (M + ROWS * G - 1) / (ROWS * G);
  if (k == KMAX)
    hipLaunchKernelGGL((filter_kernel<DT, V, KMAX, G, true>), dim3((unsigned)blocks), dim3(kFilterBlock), 0, stream,
                       logits, weights, indices, M, k);
  else
    hipLaunchKernelGGL((filter_kernel<DT, V, KMAX, G, false>), dim3((unsigned)blocks), dim3(kFilterBlock), 0, stream,
                       logits, weights, indices, M, k);
  return launch_status("tb_moe_topk_gating");
}

template <int DT, int KMAX>
static tb_status dispatch_shape(const void* logits, void* weights, int32_t* indices, int64_t M, int E, int k,
                                hipStream_t stream) {
  // Filter kernel: E = 16·V for V in {4, 8, 16} and 2 < k <= 8.  For k <= 2
  // the exact kernel's two selection rounds cost less than the filter's two
  // 16-lane sorts (measured on the fp16 E = 128, k = 2 reference grid).
  if constexpr (KMAX == 8) {
    if (E == 64) return launch_filter<DT, 4, KMAX>(logits, weights, indices, M, k, stream);
    if (E == 128) return launch_filter<DT, 8, KMAX>(logits, weights, indices, M, k, stream);
    if (E == 256) return launch_filter<DT, 16, KMAX>(logits, weights, indices, M, k, stream);
  }
  // Exact kernel: 16 elements per lane (four 16-byte loads in fp32, two in
  // fp16/bf16) and as many lanes per row as that takes.
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
