// W4A16 GEMM: Y[M, N] = fp16(A[M, K] @ dequant(W)[K, N]), fp32 accumulation.
//
// A is fp16 row-major; W is int4 in the N-packed, low-nibble-first layout with
// group-wise fp16 scales and int4 zero-points along K (see include/tbhip.h).
//
// Prefill (MFMA-bound for large M): one 256 x 256 output tile per block.  The
// dense, grouped and MoE gate/up kernels run four wavefronts, one per SIMD,
// wavefront w owning all rows and columns 64 w .. +63 as 8 x 2
// v_mfma_f32_32x32x16_f16 accumulators (tile4); the MoE down projection
// (K = I, a few K steps per tile) runs eight, two per SIMD, wavefront
// (wm, wn) owning rows 128 wm .. +127 and columns 64 wn .. +63 as 4 x 2
// accumulators (tile8), whose second wavefront per SIMD hides its short
// tiles' prologue and scatter epilogue.  A wavefront's two 32-column
// fragments are the even and the odd columns of its range: lane l owns packed
// byte l % 32 of the range, so one byte per K row carries both of its columns.
//
//   A, W  : the A tile ([256][64 halfs]), the packed W tile ([64][128 B]) and
//           the step's group of scales and zero-points stream HBM -> LDS by
//           the buffer unit (buffer_load ... lds), three stages, issued two
//           steps ahead; a wavefront waits only for its own share of the next
//           stage, and one barrier per step publishes it;
//   W     : never stored in fp16: per k16 slice one ds_read_b64_tr_b8 (the
//           gfx950 transposing LDS read) hands each lane its byte column for 8
//           consecutive k rows, and the lane dequantises in registers with the
//           standalone dequantiser's exact arithmetic ((1024 + q) and (64 + q)
//           half2 from the 0x64 / 0x54 magic numbers, exact zero-point
//           subtraction, one RNE multiply by the scale);
//   MFMA  : while the MFMAs of one slice run (16 in tile4, 8 in tile8), the
//           wavefront reads and dequantises the next slice; a step's DMAs go
//           out in four parts between the MFMAs of four slices (the first
//           part of step k + 3 after step k's barrier, the rest during step
//           k + 1), so a CU never queues a whole step's loads at once;
//   output: each lane holds 8 consecutive columns of one row per accumulator
//           group (even and odd accumulators interleaved).  The plain tile4
//           epilogue (dense and grouped GEMMs) stages the fp16 tile in LDS and
//           stores whole row runs; the MoE epilogues store 16 bytes straight
//           from the accumulators.
//   rounds: a launch of T tiles on C CUs runs ceil(T / C) rounds; when the
//           last round would be part-empty, the host may cover the last tile
//           columns with 192-row tiles instead, so that the work splits into
//           whole rounds more evenly.
// The grouped GEMM (w4a16_grouped) and the MoE layer's gate/up (moe_gate_up:
// gathered token rows, SiLU(gate) * up epilogue) and down (moe_down: routing
// weight and scatter epilogue) projections run the tile on each expert's
// operands; a last column tile of at most 128 columns runs as 256 x 128 (the
// wavefronts as 2 row groups x 2 column groups in tile4, 4 x 2 in tile8).
// Every output element sees the same MFMA operands in the same K order in
// all of them, so an expert's rows equal the dense product bit for bit.
//
// Tiles are numbered XCD-aware: consecutive hardware block ids land on
// different XCDs, so block ids are first regrouped so that each XCD owns a
// contiguous run of tiles, and runs are ordered in groups of 4 tile rows, so
// the blocks resident on one XCD share A rows and W columns in its L2.
#include "tb_common.h"
#include "prefill_plan.h"

#include <algorithm>
#include <functional>
#include <vector>
#include <mutex>
#include <type_traits>

#pragma clang fp contract(off)

namespace tb {
namespace w4a16 {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int GROUP_M = 4;  // tile rows per ordering group

struct Tile {
  int m0, n0;
};

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef int i32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t RSRC_DW3 = 0x00020000u;
constexpr uint32_t OOB = 0x80000000u;
__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, (int)RSRC_DW3);
}

// Row map of the MoE pipeline's tiles: tile row m is (token, slot) pair
// ids[m]; the pair's token is ids[m] / topk and its routing weight w[ids[m]].
struct RowMap {
  const int* ids = nullptr;
  const float* w = nullptr;
  int topk = 1;
  int pairs = 0;
};

// fp16 of an fp32 value that is already rounded: the empty asm keeps the
// conversion from being folded into the preceding multiply (a mixed-precision
// FMA would round the exact product once, not the fp32 product).
__device__ __forceinline__ _Float16 h_of_rounded(float f) {
  asm volatile("" : "+v"(f));
  return (_Float16)f;
}

// Expert and row range of grouped tile row mt: rows offsets[e] .. offsets[e+1]
// of the row space (R rows) use expert e, cut into 256-row tiles.  Offsets are
// clamped to [0, R] so that malformed ones never address rows outside A / Y.
// Returns false past the last tile.  Every wavefront searches 64 experts at a
// time, one per lane (a prefix sum of tile counts, then a ballot), so the
// search costs a few loads in flight together rather than one dependent load
// per expert.
__device__ __forceinline__ bool grouped_tile(const int* __restrict__ offsets, int experts, int R, int mt, int& e,
                                             int& m0, int& m_end) {
  const int lane = threadIdx.x & 63;
  int seen = 0;
  for (int x0 = 0; x0 < experts; x0 += 64) {
    const int x = x0 + lane;
    int lo = 0, hi = 0;
    if (x < experts) {
      lo = min(max(offsets[x], 0), R);
      hi = min(max(offsets[x + 1], lo), R);
    }
    const int cnt = (hi - lo + BM - 1) / BM;
    int incl = cnt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d);
      if (lane >= d) incl += o;
    }
    const int total = __builtin_amdgcn_readfirstlane(__shfl(incl, 63));
    if (mt < seen + total) {
      const unsigned long long hit = __ballot(seen + incl > mt);
      const int l = __builtin_ctzll(hit);
      const int lo_l = __shfl(lo, l), hi_l = __shfl(hi, l), before = seen + __shfl(incl - cnt, l);
      // uniform across the block: scalar registers, so that every address
      // derived from the tile stays scalar
      e = __builtin_amdgcn_readfirstlane(x0 + l);
      m0 = __builtin_amdgcn_readfirstlane(lo_l + (mt - before) * BM);
      m_end = __builtin_amdgcn_readfirstlane(hi_l);
      return true;
    }
    seen += total;
  }
  return false;
}

__device__ __forceinline__ int grouped_block_id() {
  const int nb = gridDim.x;
  int bid = blockIdx.x;
  if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  return bid;
}

// ---------------------------------------------------------------------------
// Decode kernel (M <= 16, HBM-bound on the weights).  A block of eight
// wavefronts owns a 256-column slab and one of S contiguous K ranges, and the
// grid never holds more blocks than the device has CUs (one block fills a CU),
// so every block starts at once.  Each wavefront streams its own contiguous
// run of 32-row units, the next unit's loads issued as soon as a unit has been
// consumed (one unit in flight per wavefront: the chip's loads then arrive
// early enough for compute to overlap them; deeper prefetch measured slower).
// Per unit a lane loads an 8 x 16 int4 block (eight 8-byte row loads; 16 lanes
// side by side cover a full 128-byte line of a row) and its A fragment; a
// group's scales and zero-points are loaded once, at the group's first unit.
// All are buffer loads whose offsets are out of range (zeros, no traffic) where
// a row, column or unit does not exist, so no load sits behind a branch and
// the compiler's wait before a unit covers only that unit.  The MFMAs
// (v_mfma_f32_16x16x32_f16, A rows >= M zero; fragment f holds columns
// 16c + f, c = lane % 16) take the codes themselves as c0 + q (c0 = 1024 for
// even columns, 64 for odd ones), built from the packed bytes by one byte
// permute per two rows and an and-or per nibble (under one VALU instruction
// per weight, against 2.4 for dequantising each weight first); the scale and
// zero-point enter once per group, in fp32:
// sum_k a (q - z) s = s (sum_k a (c0 + q) - (c0 + z) sum_k a), with the A
// row sums from one more MFMA against ones.  The weights are therefore not
// rounded to fp16 before the product (the dense and grouped kernels round
// them, as the reference dequantisation does); the difference stays far below
// the 1e-2 tolerance.  The eight wave partials are summed in LDS in a fixed
// order, so results are reproducible bit for bit.
// Across the S blocks of a slab the reduction is a serial split-K: each block
// writes its fp32 partial through to the device-coherent level, then bumps the
// slab's arrival counter; the block that arrives last reads the S partials
// (all loads in flight at once), adds them in slot order (deterministic),
// writes fp16 Y and puts the counter back to zero, so the workspace is ready
// for the next call without any clearing.
constexpr int DEC_COLS = 256, DEC_THREADS = 512, DEC_WAVES = 8, DEC_UNIT = 32, DEC_MAX_SPLITS = 16;
constexpr int AUX_SC1 = 16;  // buffer cache policy: coherent across the XCDs
// Workspace layout, the same for every shape so that calls of different shapes
// can share one buffer: [DEC_MAX_SLABS int32 arrival counters][fp32 partials].
// Counters are left at zero by every call; partials never overlap them.
constexpr int64_t DEC_MAX_SLABS = 4096;
constexpr int64_t DEC_COUNTER_BYTES = DEC_MAX_SLABS * 4;

typedef float f32x4d __attribute__((ext_vector_type(4)));

struct DecUnit {
  u32x2 w[8];  // rows kg*8 + r, columns 16c .. 16c + 15
  u32x4 a;     // A row lane % 16, k = kg*8 .. +7
};
struct DecGroup {
  u32x4 s0, s1;  // scales of the group, columns 16c .. 16c + 15
  uint32_t z0, z1;  // zero-points of the group, columns 16c .. 16c + 15
};

template <bool TAIL>
__global__ void __launch_bounds__(DEC_THREADS)
    w4a16_decode(const _Float16* __restrict__ A, const uint8_t* __restrict__ W, const _Float16* __restrict__ S,
                 const uint8_t* __restrict__ Z, _Float16* __restrict__ Y, float* __restrict__ partials,
                 int* __restrict__ counters, int M, int N, int K, int group, int splits) {
  __shared__ float part[DEC_WAVES][16 * DEC_COLS];  // 128 KiB: one partial per wavefront
  __shared__ int last_flag;
  const int slab = blockIdx.x / splits, split = blockIdx.x % splits;
  const int n0 = slab * DEC_COLS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, kg = lane >> 4;
  const int n = n0 + c * 16;
  const bool col_ok = n < N;               // at least columns n .. n+7 exist (N % 8 == 0)
  const bool col_full = n + 16 <= N;       // all 16 columns exist
  const int units = K / DEC_UNIT;
  const int u_begin = (int)((int64_t)units * split / splits), u_end = (int)((int64_t)units * (split + 1) / splits);
  const int bu = u_end - u_begin;
  const int w_begin = __builtin_amdgcn_readfirstlane(u_begin + (int)((int64_t)bu * wave / DEC_WAVES));
  const int w_end = __builtin_amdgcn_readfirstlane(u_begin + (int)((int64_t)bu * (wave + 1) / DEC_WAVES));
  const uint32_t half_n = (uint32_t)(N >> 1);
  const int arow = lane & 15;

  // Every load is a buffer load with a per-lane offset that is out of range
  // (reads zeros) where the row or column does not exist: no branches around
  // loads, so the compiler's wait before each unit covers only that unit.
  const rsrc_t rw = make_rsrc(W, (uint32_t)K * half_n);
  const rsrc_t ra = make_rsrc(A, (uint32_t)M * (uint32_t)K * 2u);
  const rsrc_t rs = make_rsrc(S, (uint32_t)(K / group) * (uint32_t)N * 2u);
  const rsrc_t rz = make_rsrc(Z, (uint32_t)(K / group) * half_n);
  const uint32_t w_off = col_full ? (uint32_t)(kg * 8) * half_n + (uint32_t)(n >> 1) : OOB;
  const uint32_t w_tail = (TAIL && col_ok && !col_full) ? (uint32_t)(kg * 8) * half_n + (uint32_t)(n >> 1) : OOB;
  const uint32_t a_off = arow < M ? ((uint32_t)arow * (uint32_t)K + (uint32_t)(kg * 8)) * 2u : OOB;
  const uint32_t s_off0 = col_ok ? (uint32_t)n * 2u : OOB, s_off1 = col_full ? (uint32_t)(n + 8) * 2u : OOB;
  const uint32_t z_off0 = col_ok ? (uint32_t)(n >> 1) : OOB, z_off1 = col_full ? (uint32_t)(n >> 1) + 4u : OOB;
  constexpr int NT = 2;  // nontemporal: the weights are read once

  f32x4d acc[16];
#pragma unroll
  for (int f = 0; f < 16; ++f) acc[f] = f32x4d{};

  // A unit past the wavefront's range is still issued, with an out-of-range
  // offset (no memory traffic, zeros): the loop has no branch around a load.
  auto load_unit = [&](DecUnit& d, int u) {
    const bool live = u < w_end;
    const uint32_t kw = live ? (uint32_t)(u * DEC_UNIT) * half_n : OOB;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      d.w[r] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rw, w_off + (uint32_t)r * half_n, kw, NT));
      if (TAIL) {
        const uint32_t t = __builtin_amdgcn_raw_buffer_load_b32(rw, w_tail + (uint32_t)r * half_n, kw, NT);
        d.w[r] = col_full ? d.w[r] : u32x2{t, 0u};
      }
    }
    d.a = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off, live ? (uint32_t)(u * DEC_UNIT) * 2u : OOB, 0);
  };
  // A group's scales and zero-points, needed only by its fold.
  auto load_group = [&](DecGroup& d, int g) {
    const uint32_t ks = (uint32_t)g * (uint32_t)N * 2u, kz = (uint32_t)g * half_n;
    d.s0 = __builtin_amdgcn_raw_buffer_load_b128(rs, s_off0, ks, 0);
    d.s1 = __builtin_amdgcn_raw_buffer_load_b128(rs, s_off1, ks, 0);
    d.z0 = __builtin_amdgcn_raw_buffer_load_b32(rz, z_off0, kz, 0);
    d.z1 = __builtin_amdgcn_raw_buffer_load_b32(rz, z_off1, kz, 0);
  };
  // One unit's MFMAs on the raw codes: B fragment f holds column 16c + f as
  // c0 + q (exact in fp16) for the lane's 8 rows, built straight from the
  // packed bytes: one byte permute takes byte b of rows 2i and 2i+1, and an
  // and-or places the two nibbles of a column under an fp16 exponent, so each
  // half2 is a k-pair of one column.  Even columns (bits 3:0) go under 0x64
  // and read 1024 + q; odd columns stay in bits 7:4 under 0x54, whose mantissa
  // unit is 1/16, and read 64 + q with no shift.  The
  // scale and zero-point are applied once per group to the fp32 sums (fold
  // below); a ninth-row MFMA against ones accumulates the A row sums it needs.
  const h8 ones = __builtin_bit_cast(h8, u32x4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u});
  auto mma_unit = [&](const DecUnit& d, f32x4d (&tmp)[16], f32x4d& asum, auto first) {
    constexpr bool FIRST = decltype(first)::value;
    const f32x4d zero{};
    const h8 af = __builtin_bit_cast(h8, d.a);
    asum = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, ones, FIRST ? zero : asum, 0, 0, 0);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      u32x4 col[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t x = d.w[2 * i][h], y = d.w[2 * i + 1][h];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const uint32_t pb = perm(y, x, (uint32_t)b | 0x0C00u | ((uint32_t)(4 + b) << 16) | 0x0C000000u);
          col[2 * b][i] = (pb & 0x000F000Fu) | 0x64006400u;      // even column: 1024 + q
          col[2 * b + 1][i] = (pb & 0x00F000F0u) | 0x54005400u;  // odd column: 64 + q (unit 1/16)
        }
      }
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) {
        const int f = h * 8 + cc;
        tmp[f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, __builtin_bit_cast(h8, col[cc]), FIRST ? zero : tmp[f],
                                                        0, 0, 0);
      }
    }
  };
  // Fold of one group: sum_k a (q - z) s = s (sum_k a (c0 + q) - (c0 + z) sum_k a),
  // c0 = 1024 for even columns f and 64 for odd ones, in fp32, for the rows
  // e < M only (rows past M are never stored).
  auto fold = [&](const f32x4d (&tmp)[16], const f32x4d& asum, const DecGroup& gp) {
#pragma unroll
    for (int f = 0; f < 16; ++f) {
      const u32x4 sv = f < 8 ? gp.s0 : gp.s1;
      const float sf = (float)__builtin_bit_cast(_Float16, (uint16_t)(sv[(f % 8) / 2] >> (16 * (f & 1))));
      const float zf = (float)((f & 1 ? 64u : 1024u) + (((f < 8 ? gp.z0 : gp.z1) >> (4 * (f % 8))) & 15u));
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (e < M) acc[f][e] = __builtin_fmaf(sf, __builtin_fmaf(-zf, asum[e], tmp[f][e]), acc[f][e]);
    }
  };

  // The wavefront's units, group by group: the group's scales and zero-points
  // are loaded at its start, its first unit starts the sums from zero, and
  // its last is followed by the fold.  The next unit's loads are issued as
  // soon as a unit's MFMAs have taken its registers (one unit in flight per
  // wavefront: double buffering measured slower, the weights' stream being
  // the limit).
  const int upg = group / DEC_UNIT;
  DecUnit buf;
  load_unit(buf, w_begin);
  int u = w_begin;
  while (u < w_end) {
    const int gend = min(w_end, (u / upg + 1) * upg);
    DecGroup gp;
    load_group(gp, u / upg);
    f32x4d tmp[16], asum;
    mma_unit(buf, tmp, asum, std::true_type{});
    load_unit(buf, ++u);
    for (; u < gend; ++u) {
      mma_unit(buf, tmp, asum, std::false_type{});
      load_unit(buf, u + 1);
    }
    fold(tmp, asum, gp);
  }

  // Accumulator f, element e: row 4 * (lane / 16) + e, column 16c + f.
#pragma unroll
  for (int f = 0; f < 16; ++f)
#pragma unroll
    for (int e = 0; e < 4; ++e) part[wave][(4 * kg + e) * DEC_COLS + c * 16 + f] = acc[f][e];
  __syncthreads();
  // Fixed-order sum of the eight wave partials; thread t owns the float4 chunks
  // t and t + 512 of the 16 x 256 tile.
  const int ncols = min(DEC_COLS, N - n0);
  constexpr int CH = 16 * DEC_COLS / 4 / DEC_THREADS;
  f32x4d red[CH];
#pragma unroll
  for (int q = 0; q < CH; ++q) {
    const int i = (threadIdx.x + q * DEC_THREADS) * 4;
    f32x4d sum = *reinterpret_cast<const f32x4d*>(&part[0][i]);
#pragma unroll
    for (int w = 1; w < DEC_WAVES; ++w) sum += *reinterpret_cast<const f32x4d*>(&part[w][i]);
    red[q] = sum;
  }
  auto store_y = [&](int q, f32x4d v) {
    const int i = (threadIdx.x + q * DEC_THREADS) * 4;
    const int m = i / DEC_COLS, cc = i % DEC_COLS;
    if (m < M && cc < ncols) {  // ncols % 8 == 0, so a chunk is all in or all out
      u32x2 h;
      h[0] = as_u32(f16x2{(_Float16)v[0], (_Float16)v[1]});
      h[1] = as_u32(f16x2{(_Float16)v[2], (_Float16)v[3]});
      *reinterpret_cast<u32x2*>(Y + (int64_t)m * N + n0 + cc) = h;
    }
  };
  if (splits == 1) {
#pragma unroll
    for (int q = 0; q < CH; ++q) store_y(q, red[q]);
    return;
  }
  // Serial split-K across the slab's blocks.  The hand-off uses the gfx950
  // (GFX942-family) memory model's encoding of agent-scope atomics rather than
  // cache-wide fences: every partial is stored and loaded with the sc1 cache
  // policy, which is how an agent-scope monotonic atomic store / load is
  // encoded (AMDGPUUsage, "Memory Model GFX942": the access is performed
  // coherently across the XCDs' separate L2s instead of in one XCD's L2).
  // Each wavefront waits for its own sc1 stores to be acknowledged
  // (s_waitcnt vmcnt(0)) before the block barrier, and only then does thread 0
  // bump the slab counter with an agent-scope atomic, so every partial of a
  // block is at the coherence point before its arrival is counted.  The block
  // that reads splits - 1 then loads the partials with sc1, which reads them
  // from that same coherence point, never from a stale line of its XCD's L2.
  // A release / acquire pair on the counter would add an L2 write-back
  // (buffer_wbl2) to every block and an invalidate to the last one; measured
  // on the box, that made the M = 1 decode about 4 us slower.
  const rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(partials, 0, 0x7FFFFFFF, (int)RSRC_DW3);
  auto poff = [&](int s2, int q) -> uint32_t {
    const int i = (threadIdx.x + q * DEC_THREADS) * 4;
    const int m = i / DEC_COLS, cc = i % DEC_COLS;
    return (m < M && cc < ncols) ? (uint32_t)((((int64_t)s2 * M + m) * N + n0 + cc) * 4) : OOB;
  };
#pragma unroll
  for (int q = 0; q < CH; ++q)
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, red[q]), rp, poff(split, q), 0, AUX_SC1);
  __builtin_amdgcn_s_waitcnt(0);  // this wavefront's partial stores acknowledged
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&counters[slab], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = (prev == splits - 1);
  }
  __syncthreads();
  if (!last_flag) return;
  u32x4 v[CH][DEC_MAX_SPLITS];
#pragma unroll
  for (int q = 0; q < CH; ++q)
#pragma unroll
    for (int s2 = 0; s2 < DEC_MAX_SPLITS; ++s2)
      if (s2 < splits && s2 != split) v[q][s2] = __builtin_amdgcn_raw_buffer_load_b128(rp, poff(s2, q), 0, AUX_SC1);
#pragma unroll
  for (int q = 0; q < CH; ++q) {
    f32x4d sum = f32x4d{};
#pragma unroll
    for (int s2 = 0; s2 < DEC_MAX_SPLITS; ++s2)
      if (s2 < splits) sum += s2 == split ? red[q] : __builtin_bit_cast(f32x4d, v[q][s2]);
    store_y(q, sum);
  }
  if (threadIdx.x == 0) __hip_atomic_store(&counters[slab], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Number of CUs of the current device, cached per device.
inline int device_cus() {
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cache[dev] = cus;
  }
  return cache[dev];
}

// One block per CU: slabs x splits never exceeds the CU count.
inline int decode_splits(int N, int K) {
  const int slabs = (N + DEC_COLS - 1) / DEC_COLS;
  const int units = K / DEC_UNIT;
  int s = device_cus() / slabs;
  s = std::min(s, DEC_MAX_SPLITS);
  s = std::min(s, units / DEC_WAVES);
  return std::max(s, 1);
}

// ---------------------------------------------------------------- dense prefill
namespace p8 {
constexpr int THREADS = 512, STAGES = 3;
constexpr int A_ST = BM * BK * 2;         // 32 KiB: [256 rows][128 B]
constexpr int W_ROWS = BK * BN / 2;       // 8 KiB:  [64 rows][128 B] packed int4
constexpr int S_OFF = W_ROWS;             // 512 B: the step's group scales, 256 fp16
constexpr int Z_OFF = S_OFF + BN * 2;     // 256 B: its zero-points (128 B) + 128 B landing pad
constexpr int PAD_OFF = Z_OFF + 256;      // 256 B: landing pad of the idle wavefronts' DMA
constexpr int W_ST = PAD_OFF + 256;       // 9 KiB per W stage
constexpr int STAGE = A_ST + W_ST;
// The plain tile4 epilogue stages its fp16 output tile in LDS (rows of
// C_STRIDE halves, a 16-byte pad) over the stages, which it no longer needs.
constexpr int C_STRIDE = BN + 8;
constexpr size_t RING_BYTES = (size_t)STAGES * STAGE;  // 123 KiB
constexpr size_t C_BYTES = (size_t)BM * C_STRIDE * 2;  // 132 KiB
constexpr size_t LDS_BYTES = RING_BYTES > C_BYTES ? RING_BYTES : C_BYTES;
static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");

typedef int v2i __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void dma16(uint32_t lds_addr, uint32_t voff, const i32x4& rsrc, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane((int)lds_addr)), "v"(voff), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane((int)soff))
               : "memory", "m0");
}
__device__ __forceinline__ void dma4(uint32_t lds_addr, uint32_t voff, const i32x4& rsrc, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane((int)lds_addr)), "v"(voff), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane((int)soff))
               : "memory", "m0");
}
// Block ids go round-robin to the 8 XCDs: regroup ids so that each XCD owns
// a contiguous run of tiles (when the count is a multiple of 8).
__device__ __forceinline__ int remap_xcd(int bid, int nb) {
  return (nb & 7) == 0 ? (bid & 7) * (nb >> 3) + (bid >> 3) : bid;
}
// Tile idx of a tiles_m x tiles_n grid of (rows x 256) tiles, in groups of
// GROUP_M tile rows (L2 reuse), columns offset by n_base.
__device__ __forceinline__ Tile tile_in_grid(int idx, int tiles_m, int tiles_n, int rows, int n_base) {
  const int per_group = GROUP_M * tiles_n;
  const int group = idx / per_group;
  const int first_m = group * GROUP_M;
  const int in_rows = min(tiles_m - first_m, GROUP_M);
  const int in_group = idx - group * per_group;
  Tile t;
  t.m0 = (first_m + in_group % in_rows) * rows;
  t.n0 = n_base + (in_group / in_rows) * BN;
  return t;
}
__device__ __forceinline__ Tile tile_of(int bid, int nb, int tiles_m, int tiles_n, int rows, int n_base) {
  return tile_in_grid(remap_xcd(bid, nb), tiles_m, tiles_n, rows, n_base);
}
__device__ __forceinline__ i32x4 rsrc4(const void* p, uint32_t bytes) {
  const uint64_t base = (uint64_t)(uintptr_t)p;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)base);
  r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32) & 0xFFFF);
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = (int)RSRC_DW3;
  return r;
}
// (x & mask) | c in one instruction: mask from a scalar register, c from a vector one
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(c));
  return r;
}

// What a tile reads and writes besides the plain product.
enum TileMode {
  T_PLAIN = 0,    // rows m < M of A and Y
  T_GATE_UP = 1,  // MoE gate/up: see below
  T_DOWN = 2      // MoE down: see below
};

// One tile at (m0, n0): the eight wavefronts as 8 / WN row groups of 32 MB
// rows times WN column groups of 64 columns.  WN = 4: 256 columns and 64 MB
// rows (MB = 4: 256, MB = 3: 192); WN = 2, MB = 2: 256 rows x 128 columns,
// for a last column tile of at most 128 columns.  Rows m < M exist; A holds
// a_rows rows.
//   T_GATE_UP: tile row m reads A row rm.ids[m] / rm.topk (a token; a bad id
//     reads zeros).  W is W13 [K, N = 2I]; the tile covers activation columns
//     a0 = n0 / 2 .. a0 + 127, and column group wn takes gate columns
//     a0 + 32 wn .. + 31 as its first 16 packed bytes and the up columns of the
//     same activation columns (I + ...) as its last 16, so a lane ends with
//     the gate and the up sum of the same activation columns (accumulator
//     elements 4g + e and 4(g + 2) + e).  Y [M, I] gets fp16(silu(g) * u) of
//     the fp16-rounded gate and up values.
//   T_DOWN: row m's fp32 sums are multiplied by rm.w[rm.ids[m]], rounded once
//     to fp16 and stored at row rm.ids[m] of Y (rows with a bad id are not
//     stored).
template <int MB, int WN = 4, int MODE = T_PLAIN>
__device__ __forceinline__ void tile8(uint8_t* __restrict__ lds, const _Float16* __restrict__ A,
                                      const uint8_t* __restrict__ W, const _Float16* __restrict__ S,
                                      const uint8_t* __restrict__ Z, _Float16* __restrict__ Y, int M, int N, int K,
                                      int group, const Tile tile, int a_rows = -1, const RowMap rm = RowMap{}) {
  static_assert((WN == 4 && (MB == 3 || MB == 4)) || (WN == 2 && MB == 2), "tile8 shapes");
  if (MODE == T_PLAIN) a_rows = M;
  constexpr int TM = 32 * MB * (8 / WN);  // tile rows
  constexpr int AI = TM / 64;             // A DMA instructions per wavefront and step (8 rows each)
  constexpr int DMA_PER_STEP = AI + 5;
  const int t = threadIdx.x, lane = t & 63, h = lane >> 5, j = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = w / WN, wn = w % WN;
  const int nk = K / BK;
  const uint32_t half_n = (uint32_t)(N / 2);

  const i32x4 ra = rsrc4(A, (uint32_t)a_rows * (uint32_t)K * 2u);
  const int I = N / 2, a0 = tile.n0 / 2;  // T_GATE_UP: activation columns
  const i32x4 rw = rsrc4(W, (uint32_t)K * half_n);
  const i32x4 rs = rsrc4(S, (uint32_t)(K / group) * (uint32_t)N * 2u);
  const i32x4 rz = rsrc4(Z, (uint32_t)(K / group) * half_n);

  // A DMA: instruction i of wavefront w fills rows 8 (AI w + i) .. +7 (lane
  // L: row + L / 8, 16-byte slot L % 8, which holds chunk slot ^ swizzle).
  uint32_t a_off[AI];
#pragma unroll
  for (int i = 0; i < AI; ++i) {
    const int row = 8 * (AI * w + i) + (lane >> 3);
    const int c = (lane & 7) ^ ((row ^ (row >> 3)) & 7);
    const int m = tile.m0 + row;
    int src = m;
    if (MODE == T_GATE_UP && m < M) {
      const int pid = rm.ids[m];
      src = (unsigned)pid < (unsigned)rm.pairs ? pid / rm.topk : a_rows;
    }
    a_off[i] = m < M && src < a_rows ? ((uint32_t)src * (uint32_t)K + (uint32_t)c * 8u) * 2u : OOB;
  }
  // W DMA: instruction i of wavefront w fills rows 8w + 2i, +1 (lane L: row +
  // L / 32, dword L % 32 of the row, i.e. 16-byte slot (L % 32) / 4, which
  // holds chunk slot ^ (row & 7)).
  uint32_t w_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 8 * w + 2 * i + (lane >> 5);
    const int c = ((lane & 31) >> 2) ^ (r & 7);
    if (MODE == T_GATE_UP) {
      // chunk c: gate (c even) or up (c odd) of activation columns a0 + 32 (c / 2) ..,
      // this dword their 8 columns from a0 + 32 (c / 2) + 8 (lane % 4)
      const int acol = a0 + 32 * (c >> 1) + 8 * (lane & 3);
      const uint32_t byte = (uint32_t)((c & 1) * (I / 2) + acol / 2);
      w_off[i] = acol < I ? (uint32_t)r * half_n + byte : OOB;
    } else {
      const uint32_t col = (uint32_t)(tile.n0 / 2 + c * 16 + (lane & 3) * 4);
      w_off[i] = col < half_n ? (uint32_t)r * half_n + col : OOB;
    }
  }
  // Scales and zero-points of a step's group: wavefronts 0 and 1 fetch the
  // 512 scale bytes, wavefront 2 the 128 zero-point bytes (lanes 32..63 land
  // in the pad), the others nothing (their lanes land in the pad).
  uint32_t sz_off = OOB, sz_lds = PAD_OFF;
  const i32x4& rsz = w == 2 ? rz : rs;
  if (w < 2) {
    if (MODE == T_GATE_UP) {
      // scale slot t = 128 w + 2 lane (two columns) of column group t / 64:
      // gate (t % 64 < 32) or up of activation column a0 + 32 (t / 64) + t % 32
      const int t2 = 128 * w + 2 * lane, acol = a0 + 32 * (t2 >> 6) + (t2 & 31);
      sz_off = acol < I ? (uint32_t)(((t2 & 32) ? I : 0) + acol) * 2u : OOB;
    } else {
      const uint32_t col = (uint32_t)tile.n0 + (uint32_t)(w * 128 + lane * 2);
      sz_off = col < (uint32_t)N ? col * 2u : OOB;
    }
    sz_lds = S_OFF + w * 256;
  } else if (w == 2) {
    if (MODE == T_GATE_UP) {
      // zero-point bytes b = 4 lane .. + 3 of column group b / 32: gate
      // (b % 32 < 16) or up bytes of activation columns a0 + 32 (b / 32) + 2 (b % 16) ..
      const int b = 4 * lane, acol = a0 + 32 * (b >> 5) + 2 * (b & 15);
      sz_off = lane < 32 && acol < I ? (uint32_t)(((b & 16) ? I / 2 : 0) + acol / 2) : OOB;
    } else {
      const uint32_t col = (uint32_t)(tile.n0 / 2 + lane * 4);
      sz_off = lane < 32 && col < half_n ? col : OOB;
    }
    sz_lds = Z_OFF;
  }
  const uint32_t lds0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)(
      __attribute__((address_space(3))) void*)lds);

  // DMA of step ks into stage st (out-of-range offsets past the last step:
  // nothing is read, the stage is not used again).
  // DMA instruction d (0 .. 8) of step ks into stage st
  // past the last step the DMAs read through an empty resource (zeros, no
  // traffic): a scalar select instead of a per-lane one
  auto live_rsrc = [](bool live, i32x4 r) __attribute__((always_inline)) {
    r[2] = __builtin_amdgcn_readfirstlane(live ? r[2] : 0);
    return r;
  };
  auto issue_one = [&](int ks, int st, int d) __attribute__((always_inline)) {
    const bool live = ks < nk;
    const uint32_t sb = lds0 + (uint32_t)(st * STAGE);
    if (d < AI) {
      dma16(sb + (uint32_t)(8 * (AI * w + d) * 128), a_off[d], live_rsrc(live, ra), (uint32_t)(ks * BK) * 2u);
    } else if (d < AI + 4) {
      dma4(sb + (uint32_t)(A_ST + (8 * w + 2 * (d - AI)) * 128), w_off[d - AI], live_rsrc(live, rw),
           (uint32_t)(ks * BK) * half_n);
    } else {
      const uint32_t g = (uint32_t)(ks * BK) / (uint32_t)group;
      const uint32_t ss = w == 2 ? g * half_n : g * (uint32_t)N * 2u;
      dma4(sb + (uint32_t)A_ST + sz_lds, sz_off, live_rsrc(live, rsz), ss);
    }
  };
  auto issue = [&](int ks, int st) __attribute__((always_inline)) {
    const bool live = ks < nk;
    const uint32_t sb = lds0 + (uint32_t)(st * STAGE);
    const uint32_t sa = (uint32_t)(ks * BK) * 2u;
#pragma unroll
    for (int i = 0; i < AI; ++i) dma16(sb + (uint32_t)(8 * (AI * w + i) * 128), a_off[i], live_rsrc(live, ra), sa);
    const uint32_t sw = (uint32_t)(ks * BK) * half_n;
#pragma unroll
    for (int i = 0; i < 4; ++i) dma4(sb + (uint32_t)(A_ST + (8 * w + 2 * i) * 128), w_off[i], live_rsrc(live, rw), sw);
    const uint32_t g = (uint32_t)(ks * BK) / (uint32_t)group;
    const uint32_t ss = w == 2 ? g * half_n : g * (uint32_t)N * 2u;
    dma4(sb + (uint32_t)A_ST + sz_lds, sz_off, live_rsrc(live, rsz), ss);
  };

  // A fragment mb of slice c: row 32 (MB wm + mb) + j, chunk 2c + h; its
  // swizzle depends on the row's 32-row block through bit 2 only (parity
  // of MB wm + mb).
  uint32_t fa_off[4][2];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int sw = (j ^ (4 * par + (j >> 3))) & 7;
      fa_off[c][par] = (uint32_t)(wm * MB * 4096 + j * 128 + (((2 * c + h) ^ sw) << 4));
    }
  // Transposing byte read of slice c: lane p = 2r + b of its group of 16
  // (group G = lane / 16: columns 16 (G & 1) .., rows 8 (G >> 1) ..) points at
  // row 16c + 8 (G >> 1) + pi(r), bytes 32 wn + 16 (G & 1) + 8b .. +7, where
  // pi swaps 1 <-> 2 and 5 <-> 6: byte r of the result then holds row pi(r),
  // so each dword reads rows (0, 2, 1, 3) and a k-row pair sits in bytes 0 and
  // 2 (or, shifted down by 8, in bytes 1 and 3) with no byte permute.
  uint32_t wt_off;
  {
    const int p = lane & 15, r = p >> 1, b = p & 1, G = lane >> 4;
    const int pr = (r & 4) | ((r & 1) << 1) | ((r >> 1) & 1);
    const int cb = 2 * wn + (G & 1);
    wt_off = (uint32_t)(A_ST + (8 * (G >> 1) + pr) * 128 + ((cb ^ pr) << 4) + 8 * b);
  }

  f32x16 acc[MB][2];

  // T_DOWN: the pair id of each of the lane's rows now, its routing weight
  // after the prologue, so that neither load's latency lands in the epilogue
  int row_pid[MODE == T_DOWN ? MB : 1];
  float row_w[MODE == T_DOWN ? MB : 1];
  if (MODE == T_DOWN) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int m = tile.m0 + 32 * (MB * wm + mb) + j;
      row_pid[mb] = m < M ? rm.ids[m] : -1;
    }
  }
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i][0] = acc[i][1] = f32x16{};

  // magic-number words in registers (a VOP3 instruction takes one scalar operand)
  const uint32_t c64 = __builtin_amdgcn_readfirstlane(0x64006400u) + (uint32_t)(lane >> 6);
  const uint32_t c54 = __builtin_amdgcn_readfirstlane(0x54005400u) + (uint32_t)(lane >> 6);
  h8 fa[2][MB];
  h8 wf[2][2];
  uint32_t sE = 0, sO = 0, zE = 0, zO = 0;  // half2 {s, s} / {1024 + z, 1024 + z} / {64 + z, 64 + z}

  auto load_scales = [&](int st) __attribute__((always_inline)) {
    const uint8_t* sb = lds + st * STAGE + A_ST;
    const uint32_t s2 = *reinterpret_cast<const uint32_t*>(sb + S_OFF + (wn * 64 + 2 * j) * 2);
    const uint32_t zb = sb[Z_OFF + wn * 32 + j];
    sE = perm(s2, s2, 0x01000100u);
    sO = perm(s2, s2, 0x03020302u);
    const uint32_t zz = zb | (zb << 16);
    zE = (zz & 0x000F000Fu) | 0x64006400u;
    zO = (zz & 0x00F000F0u) | 0x54005400u;
  };
  auto read_a = [&](int st, int c, int buf, int mb) __attribute__((always_inline)) {
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    lds_u8* const base = (lds_u8*)(__attribute__((address_space(3))) void*)lds;
    fa[buf][mb] = *(__attribute__((address_space(3))) const h8*)(base + fa_off[c][(MB * wm + mb) & 1] +
                                                                   (st * STAGE + mb * 4096));
  };
  auto read_w = [&](int st, int c) __attribute__((always_inline)) -> v2i {
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    lds_u8* const base = (lds_u8*)(__attribute__((address_space(3))) void*)lds;
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        (__attribute__((address_space(3))) v2i*)(base + st * STAGE + c * 2048 + wt_off));
  };
  // k-row pair (2q, 2q + 1) in bytes 0 and 2 of a word; the even column's
  // nibbles under 0x64 read 1024 + q, the odd column's (bits 7:4) under 0x54
  // read 64 + q (the masks ignore bytes 1 and 3).
  auto dequant_pair = [&](const v2i x, int buf, int q, u32x4& e, u32x4& o) __attribute__((always_inline)) {
    const uint32_t src = (uint32_t)x[q >> 1];
    const uint32_t d = (q & 1) ? src >> 8 : src;  // k rows 2q, 2q + 1 in bytes 0 and 2
    e[q] = as_u32((as_h2(and_or(d, 0x000F000Fu, c64)) - as_h2(zE)) * as_h2(sE));
    o[q] = as_u32((as_h2(and_or(d, 0x00F000F0u, c54)) - as_h2(zO)) * as_h2(sO));
  };

  // A step's DMAs go out in four parts, one per slice, so that the eight
  // wavefronts of a CU never queue a whole step's loads at the texture unit at
  // once: part 0 (PA instructions) of step kt + 3 in the slice after step kt's
  // barrier (stage kt % 3 is free from that barrier on), parts 1..3 (PB each)
  // in slices 1..3 of step kt + 1, before its barrier.  At a barrier the
  // outstanding loads are then the next step's whole stage, DMA_PER_STEP of
  // them, as before.
  constexpr int NQ = 2 * MB;
  constexpr int PB = DMA_PER_STEP / 4, PA = DMA_PER_STEP - 3 * PB;
  constexpr int DMA_GAP = NQ / (PA > PB ? PA : PB);  // MFMAs between two DMAs of a part
  static_assert(DMA_GAP >= 1 && (PA - 1) * DMA_GAP < NQ && (PB - 1) * DMA_GAP < NQ, "DMA slots");
  // vmcnt(n) with lgkmcnt(0) (vmcnt is split: bits 3:0 and 15:14)
  constexpr int VM1 = DMA_PER_STEP, VM2 = DMA_PER_STEP + PA;
  constexpr int WAIT_BAR = (VM1 & 15) | ((VM1 >> 4) << 14) | (7 << 4) | (0 << 8);
  constexpr int WAIT_PRO = (VM2 & 15) | ((VM2 >> 4) << 14) | (7 << 4) | (0 << 8);
  // The barrier: the compiler may not move LDS accesses across it (the empty
  // asm is a compiler memory barrier); no wait beyond the explicit one.
  auto barrier = [&]() __attribute__((always_inline)) {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // prologue: steps 0 and 1 and part 0 of step 2 in flight (its other parts go
  // out in step 0), step 0 landed, slice 0 read
  issue(0, 0);
  issue(1, 1);
#pragma unroll
  for (int d = 0; d < PA; ++d) issue_one(2, 2, d);
  __builtin_amdgcn_s_waitcnt(WAIT_PRO);
  barrier();
  load_scales(0);
  if (MODE == T_DOWN) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      row_w[mb] = (unsigned)row_pid[mb] < (unsigned)rm.pairs ? rm.w[row_pid[mb]] : 0.f;
  }
  v2i xs[4];
  {
#pragma unroll
    for (int c = 0; c < 4; ++c) xs[c] = read_w(0, c);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) read_a(0, 0, 0, mb);
    u32x4 e, o;
#pragma unroll
    for (int q = 0; q < 4; ++q) dequant_pair(xs[0], 0, q, e, o);
    wf[0][0] = __builtin_bit_cast(h8, e);
    wf[0][1] = __builtin_bit_cast(h8, o);
  }

  // One k16 slice: 8 MFMAs on buffer `cur`; the next slice (nst, cn) read
  // into the other buffer while they run: its A fragments, then its
  // dequantisation from the byte column xs[cn].  The slice after each
  // barrier (cn == 0) also reads the byte columns of all four slices of the
  // new stage, slice 0's first, so later slices never wait on them.
  // (After the last step the reads go to a stage that is not used again.)
  auto slice = [&](int cur, int nst, int cn, auto body) __attribute__((always_inline)) {
    u32x4 e, o;
#pragma unroll
    for (int q = 0; q < 2 * MB; ++q) {
      const int mb = q >> 1, nb = q & 1;
      acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[cur][nb], fa[cur][mb], acc[mb][nb], 0, 0, 0);
      if (cn == 0 && q == 0) xs[0] = read_w(nst, 0);
      if (q >= 1 && q < MB + 1) read_a(nst, cn, cur ^ 1, q - 1);
      if (cn == 0 && q >= 2 * MB - 3) xs[q - 2 * MB + 4] = read_w(nst, q - 2 * MB + 4);
#pragma unroll
      for (int dq = 0; dq < 4; ++dq)
        if (q == (MB >= 3 ? MB - 1 + dq : 1 + dq / 2)) dequant_pair(xs[cn], cur ^ 1, dq, e, o);
      body(q);
      __builtin_amdgcn_sched_barrier(0);
    }
    wf[cur ^ 1][0] = __builtin_bit_cast(h8, e);
    wf[cur ^ 1][1] = __builtin_bit_cast(h8, o);
  };

  // Step kt on stage ST = kt % 3 (a compile-time constant in each unrolled copy).
  auto step = [&](int kt, auto stc) __attribute__((always_inline)) {
    constexpr int ST = decltype(stc)::value;
    constexpr int NST = (ST + 1) % 3, PST = (ST + 2) % 3;
    // parts 1..3 of step kt + 2 into stage PST (free since step kt - 1's barrier)
    auto part = [&](int jp) __attribute__((always_inline)) {
      return [&, jp](int q) __attribute__((always_inline)) {
        if (q % DMA_GAP == 0 && q / DMA_GAP < PB) issue_one(kt + 2, PST, PA + (jp - 1) * PB + q / DMA_GAP);
      };
    };
    slice(0, ST, 1, part(1));
    slice(1, ST, 2, part(2));
    if (w >= 4) __builtin_amdgcn_s_setprio(0);
    slice(0, ST, 3, part(3));
    // step kt + 1 landed (each wavefront waits for its own DMA, only step
    // kt + 2's may still be in flight; the barrier publishes all of them) and
    // every wavefront has its stage-ST fragments in registers
    __builtin_amdgcn_s_waitcnt(WAIT_BAR);
    barrier();
    // The two wavefronts of a SIMD (w, w + 4) share its issue; by age the
    // older one would run ahead and wait at the barrier while the younger
    // finishes alone.  The younger one leads the three slices after each
    // barrier, the older one the last, so both arrive together.
    if (w >= 4) __builtin_amdgcn_s_setprio(1);
    load_scales(NST);
    // part 0 of step kt + 3 into stage ST (free from this barrier on)
    slice(1, NST, 0, [&](int q) {
      if (q % DMA_GAP == 0 && q / DMA_GAP < PA) issue_one(kt + 3, ST, q / DMA_GAP);
    });
  };
  int kt = 0;
  for (; kt + 2 < nk; kt += 3) {
    step(kt, std::integral_constant<int, 0>{});
    step(kt + 1, std::integral_constant<int, 1>{});
    step(kt + 2, std::integral_constant<int, 2>{});
  }
  if (kt < nk) step(kt, std::integral_constant<int, 0>{});
  if (kt + 1 < nk) step(kt + 1, std::integral_constant<int, 1>{});
  __builtin_amdgcn_s_waitcnt(0);

  // Epilogue: element 4g + e of accumulator (mb, nb) is row 32 (MB wm + mb) + j,
  // column 64 wn + 16 g + 8 h + 2 e + nb of the tile.
  if (MODE == T_GATE_UP) {
    // g = 0, 1: gate of activation columns a0 + 32 wn + 16 g + 8 h + 2 e + nb;
    // g + 2: up of the same columns
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int m = tile.m0 + 32 * (MB * wm + mb) + j;
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int acol = a0 + 32 * wn + 16 * g + 8 * h;
        u32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          _Float16 r[2];
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) {
            const float gv = (float)(_Float16)acc[mb][nb][4 * g + e];
            const float uv = (float)(_Float16)acc[mb][nb][4 * (g + 2) + e];
            float sg = 1.0f + expf(-gv);
            asm volatile("" : "+v"(sg));
            r[nb] = h_of_rounded(gv / sg * uv);
          }
          v[e] = as_u32(f16x2{r[0], r[1]});
        }
        if (m < M && acol < I) *reinterpret_cast<u32x4*>(Y + (int64_t)m * I + acol) = v;
      }
    }
    return;
  }
  const int col0 = tile.n0 + 64 * wn + 8 * h;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = tile.m0 + 32 * (MB * wm + mb) + j;
    int64_t dst = m;
    float rw = 1.f;
    if (MODE == T_DOWN) {
      dst = row_pid[mb];
      rw = row_w[mb];
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = col0 + 16 * g;
      u32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (MODE == T_DOWN)
          v[e] = as_u32(f16x2{h_of_rounded(acc[mb][0][4 * g + e] * rw), h_of_rounded(acc[mb][1][4 * g + e] * rw)});
        else
          v[e] = as_u32(f16x2{(_Float16)acc[mb][0][4 * g + e], (_Float16)acc[mb][1][4 * g + e]});
      }
      const bool ok = MODE == T_DOWN ? (unsigned)dst < (unsigned)rm.pairs : m < M;
      if (ok && n < N) *reinterpret_cast<u32x4*>(Y + dst * N + n) = v;
    }
  }
}
// Four-wavefront tile (one wavefront per SIMD).  WN = 4: 32 MB rows (MB = 8:
// 256, MB = 6: 192) x 256 columns, wavefront w owning all rows and columns
// 64 w .. 64 w + 63 as MB x 2 accumulators (up to 256 accumulator
// registers), so each W fragment is dequantised once per block rather than by
// the two wavefronts that share it in tile8 (half the VALU work, and under
// the power cap a higher clock).  WN = 2, MB = 4: 256 rows x 128 columns, the
// wavefronts as 2 row groups x 2 column groups, for a last column tile of at
// most 128 columns.  Modes, rows and a_rows as in tile8.  A lone wavefront cannot hide its own stalls behind another
// one, so every operation of the next slice is placed between this slice's
// MFMAs: the A fragments one after each of the first MB MFMAs, and each k-row
// pair's dequantisation as three stages (and-or, subtract, multiply) one MFMA
// apart, each pinned in place (the compiler would otherwise sink them to the
// slice's end, where they stall the next slice's first MFMA).  Same LDS
// stages, DMA, fragment layout and MFMA operands as tile8, so the results are
// bit-identical to it.
template <int MB, int WN = 4, int MODE = T_PLAIN>
__device__ __forceinline__ void tile4(uint8_t* __restrict__ lds, const _Float16* __restrict__ A,
                                      const uint8_t* __restrict__ W, const _Float16* __restrict__ S,
                                      const uint8_t* __restrict__ Z, _Float16* __restrict__ Y, int M, int N, int K,
                                      int group, const Tile tile, int a_rows = -1, const RowMap rm = RowMap{}) {
  static_assert((WN == 4 && (MB == 8 || MB == 6)) || (WN == 2 && MB == 4), "tile4 shapes");
  if (MODE == T_PLAIN) a_rows = M;
  constexpr int TM = 32 * MB * (4 / WN);  // tile rows
  constexpr int AI = TM / 32;  // A DMA instructions per wavefront and step (8 rows each, 4 wavefronts)
  constexpr int WI = 8;        // W DMA instructions per wavefront and step (2 rows each)
  constexpr int DMA_PER_STEP = AI + WI + 1;
  constexpr int NQ = 2 * MB;   // MFMAs per slice
  const int t = threadIdx.x, lane = t & 63, h = lane >> 5, j = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = w / WN, wn = w % WN;
  const int nk = K / BK;
  const uint32_t half_n = (uint32_t)(N / 2);
  const int I = N / 2, a0 = tile.n0 / 2;  // T_GATE_UP: activation columns

  const i32x4 ra = rsrc4(A, (uint32_t)a_rows * (uint32_t)K * 2u);
  const i32x4 rw = rsrc4(W, (uint32_t)K * half_n);
  const i32x4 rs = rsrc4(S, (uint32_t)(K / group) * (uint32_t)N * 2u);
  const i32x4 rz = rsrc4(Z, (uint32_t)(K / group) * half_n);
  // past the last step the DMAs go through empty resources (zeros, no traffic)
  auto live_rsrc = [](bool live, i32x4 r) __attribute__((always_inline)) {
    r[2] = __builtin_amdgcn_readfirstlane(live ? r[2] : 0);
    return r;
  };

  // A DMA: instruction i of wavefront w fills rows 8 (AI w + i) .. +7
  uint32_t a_off[AI];
#pragma unroll
  for (int i = 0; i < AI; ++i) {
    const int row = 8 * (AI * w + i) + (lane >> 3);
    const int c = (lane & 7) ^ ((row ^ (row >> 3)) & 7);
    const int m = tile.m0 + row;
    int src = m;
    if (MODE == T_GATE_UP && m < M) {
      const int pid = rm.ids[m];
      src = (unsigned)pid < (unsigned)rm.pairs ? pid / rm.topk : a_rows;
    }
    a_off[i] = m < M && src < a_rows ? ((uint32_t)src * (uint32_t)K + (uint32_t)c * 8u) * 2u : OOB;
  }
  // W DMA: instruction i of wavefront w fills rows 16 w + 2 i, +1 (lane L: row
  // + L / 32, dword L % 32, 16-byte slot (L % 32) / 4 holding chunk slot ^ (row & 7))
  uint32_t w_off[WI];
#pragma unroll
  for (int i = 0; i < WI; ++i) {
    const int r = 16 * w + 2 * i + (lane >> 5);
    const int c = ((lane & 31) >> 2) ^ (r & 7);
    if (MODE == T_GATE_UP) {
      // chunk c: gate (c even) or up (c odd) of activation columns a0 + 32 (c / 2) ..,
      // this dword their 8 columns from a0 + 32 (c / 2) + 8 (lane % 4)
      const int acol = a0 + 32 * (c >> 1) + 8 * (lane & 3);
      const uint32_t byte = (uint32_t)((c & 1) * (I / 2) + acol / 2);
      w_off[i] = acol < I ? (uint32_t)r * half_n + byte : OOB;
    } else {
      const uint32_t col = (uint32_t)(tile.n0 / 2 + c * 16 + (lane & 3) * 4);
      w_off[i] = col < half_n ? (uint32_t)r * half_n + col : OOB;
    }
  }
  uint32_t sz_off = OOB, sz_lds = PAD_OFF;
  const bool zw = w == 2;
  if (w < 2) {
    if (MODE == T_GATE_UP) {
      // scale slot t = 128 w + 2 lane (two columns) of column group t / 64:
      // gate (t % 64 < 32) or up of activation column a0 + 32 (t / 64) + t % 32
      const int t2 = 128 * w + 2 * lane, acol = a0 + 32 * (t2 >> 6) + (t2 & 31);
      sz_off = acol < I ? (uint32_t)(((t2 & 32) ? I : 0) + acol) * 2u : OOB;
    } else {
      const uint32_t col = (uint32_t)tile.n0 + (uint32_t)(w * 128 + lane * 2);
      sz_off = col < (uint32_t)N ? col * 2u : OOB;
    }
    sz_lds = S_OFF + w * 256;
  } else if (w == 2) {
    if (MODE == T_GATE_UP) {
      // zero-point bytes b = 4 lane .. + 3 of column group b / 32: gate
      // (b % 32 < 16) or up bytes of activation columns a0 + 32 (b / 32) + 2 (b % 16) ..
      const int b = 4 * lane, acol = a0 + 32 * (b >> 5) + 2 * (b & 15);
      sz_off = lane < 32 && acol < I ? (uint32_t)(((b & 16) ? I / 2 : 0) + acol / 2) : OOB;
    } else {
      const uint32_t col = (uint32_t)(tile.n0 / 2 + lane * 4);
      sz_off = lane < 32 && col < half_n ? col : OOB;
    }
    sz_lds = Z_OFF;
  }
  const uint32_t lds0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)(
      __attribute__((address_space(3))) void*)lds);

  auto issue_one = [&](int ks, int st, int d) __attribute__((always_inline)) {
    const bool live = ks < nk;
    const uint32_t sb = lds0 + (uint32_t)(st * STAGE);
    if (d < AI) {
      dma16(sb + (uint32_t)(8 * (AI * w + d) * 128), a_off[d], live_rsrc(live, ra), (uint32_t)(ks * BK) * 2u);
    } else if (d < AI + WI) {
      dma4(sb + (uint32_t)(A_ST + (16 * w + 2 * (d - AI)) * 128), w_off[d - AI], live_rsrc(live, rw),
           (uint32_t)(ks * BK) * half_n);
    } else {
      const uint32_t g = (uint32_t)(ks * BK) / (uint32_t)group;
      const uint32_t ss = zw ? g * half_n : g * (uint32_t)N * 2u;
      dma4(sb + (uint32_t)A_ST + sz_lds, sz_off, live_rsrc(live, zw ? rz : rs), ss);
    }
  };

  uint32_t fa_off[4][2];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int sw = (j ^ (4 * par + (j >> 3))) & 7;
      fa_off[c][par] = (uint32_t)(wm * MB * 4096 + j * 128 + (((2 * c + h) ^ sw) << 4));
    }
  uint32_t wt_off;
  {
    const int p = lane & 15, r = p >> 1, b = p & 1, G = lane >> 4;
    const int pr = (r & 4) | ((r & 1) << 1) | ((r >> 1) & 1);
    const int cb = 2 * wn + (G & 1);
    wt_off = (uint32_t)(A_ST + (8 * (G >> 1) + pr) * 128 + ((cb ^ pr) << 4) + 8 * b);
  }

  f32x16 acc[MB][2];
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i][0] = acc[i][1] = f32x16{};

  // T_DOWN: the pair id of each of the lane's rows now, its routing weight
  // after the prologue, so that neither load's latency lands in the epilogue
  int row_pid[MODE == T_DOWN ? MB : 1];
  float row_w[MODE == T_DOWN ? MB : 1];
  if (MODE == T_DOWN) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int m = tile.m0 + 32 * (MB * wm + mb) + j;
      row_pid[mb] = m < M ? rm.ids[m] : -1;
    }
  }

  const uint32_t c64 = __builtin_amdgcn_readfirstlane(0x64006400u) + (uint32_t)(lane >> 6);
  const uint32_t c54 = __builtin_amdgcn_readfirstlane(0x54005400u) + (uint32_t)(lane >> 6);
  h8 fa[2][MB];
  h8 wf[2][2];
  uint32_t sE = 0, sO = 0, zE = 0, zO = 0;

  auto load_scales = [&](int st) __attribute__((always_inline)) {
    const uint8_t* sb = lds + st * STAGE + A_ST;
    const uint32_t s2 = *reinterpret_cast<const uint32_t*>(sb + S_OFF + (wn * 64 + 2 * j) * 2);
    const uint32_t zb = sb[Z_OFF + wn * 32 + j];
    sE = perm(s2, s2, 0x01000100u);
    sO = perm(s2, s2, 0x03020302u);
    const uint32_t zz = zb | (zb << 16);
    zE = (zz & 0x000F000Fu) | 0x64006400u;
    zO = (zz & 0x00F000F0u) | 0x54005400u;
  };
  auto read_a = [&](int st, int c, int buf, int mb) __attribute__((always_inline)) {
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    lds_u8* const base = (lds_u8*)(__attribute__((address_space(3))) void*)lds;
    fa[buf][mb] = *(__attribute__((address_space(3))) const h8*)(base + fa_off[c][(MB * wm + mb) & 1] +
                                                                   (st * STAGE + mb * 4096));
  };
  auto read_w = [&](int st, int c) __attribute__((always_inline)) -> v2i {
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    lds_u8* const base = (lds_u8*)(__attribute__((address_space(3))) void*)lds;
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        (__attribute__((address_space(3))) v2i*)(base + st * STAGE + c * 2048 + wt_off));
  };
  auto dequant_pair = [&](const v2i x, int q, u32x4& e, u32x4& o) __attribute__((always_inline)) {
    const uint32_t src = (uint32_t)x[q >> 1];
    const uint32_t d = (q & 1) ? src >> 8 : src;
    e[q] = as_u32((as_h2(and_or(d, 0x000F000Fu, c64)) - as_h2(zE)) * as_h2(sE));
    o[q] = as_u32((as_h2(and_or(d, 0x00F000F0u, c54)) - as_h2(zO)) * as_h2(sO));
  };

  // A step's DMAs go out in four parts, one per slice, so that the four
  // wavefronts of a CU never queue a whole step's loads at the texture unit at
  // once: part 0 (PA instructions) of step kt + 3 in the slice after step kt's
  // barrier (stage kt % 3 is free from that barrier on), parts 1..3 (PB each)
  // in slices 1..3 of step kt + 1, before its barrier.  At a barrier the
  // outstanding loads are then the next step's whole stage, DMA_PER_STEP of
  // them, as before.
  constexpr int PB = DMA_PER_STEP / 4, PA = DMA_PER_STEP - 3 * PB;
  constexpr int DMA_GAP = NQ / (PA > PB ? PA : PB);  // MFMAs between two DMAs of a part
  static_assert(DMA_GAP >= 1 && (PA - 1) * DMA_GAP < NQ && (PB - 1) * DMA_GAP < NQ, "DMA slots");
  constexpr int VM1 = DMA_PER_STEP, VM2 = DMA_PER_STEP + PA;
  constexpr int WAIT_BAR = (VM1 & 15) | ((VM1 >> 4) << 14) | (7 << 4) | (0 << 8);
  constexpr int WAIT_PRO = (VM2 & 15) | ((VM2 >> 4) << 14) | (7 << 4) | (0 << 8);
  auto barrier = [&]() __attribute__((always_inline)) {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // stages 0 and 1 whole, part 0 of stage 2 (its other parts go out in step 0)
#pragma unroll
  for (int st = 0; st < 3; ++st)
#pragma unroll
    for (int d = 0; d < (st < 2 ? DMA_PER_STEP : PA); ++d) issue_one(st, st, d);
  __builtin_amdgcn_s_waitcnt(WAIT_PRO);
  barrier();
  load_scales(0);
  if (MODE == T_DOWN) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      row_w[mb] = (unsigned)row_pid[mb] < (unsigned)rm.pairs ? rm.w[row_pid[mb]] : 0.f;
  }
  v2i xs[4];
  {
#pragma unroll
    for (int c = 0; c < 4; ++c) xs[c] = read_w(0, c);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) read_a(0, 0, 0, mb);
    u32x4 e, o;
#pragma unroll
    for (int q = 0; q < 4; ++q) dequant_pair(xs[0], q, e, o);
    wf[0][0] = __builtin_bit_cast(h8, e);
    wf[0][1] = __builtin_bit_cast(h8, o);
  }

  // One k16 slice: 2 MB MFMAs on buffer `cur`, one operation of the next
  // slice after each: its A fragments first, its dequantisation (one k-row
  // pair every other MFMA) last.  The slice after a barrier (cn == 0) also
  // reads the byte columns of the new stage's four slices.
  auto slice = [&](int cur, int nst, int cn, auto body) __attribute__((always_inline)) {
    u32x4 e, o;
    uint32_t ae[4], ao[4], se[4], so[4];
    // k-row pair p's dequantisation in three pinned stages one MFMA apart:
    // and-or at slot SA + SP p, subtract one slot later, multiply two slots later
    constexpr int SA = NQ >= 12 ? NQ - 10 : 1, SP = NQ >= 12 ? 2 : 1;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int mb = q >> 1, nb = q & 1;
      acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[cur][nb], fa[cur][mb], acc[mb][nb], 0, 0, 0);
      if (cn == 0 && q == 0) xs[0] = read_w(nst, 0);
      if (q >= 1 && q <= MB) read_a(nst, cn, cur ^ 1, q - 1);
      if (cn == 0 && q >= MB + 1 && q <= MB + 3) xs[q - MB] = read_w(nst, q - MB);
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        if (q == SA + SP * pp) {
          const uint32_t src = (uint32_t)xs[cn][pp >> 1];
          const uint32_t d = (pp & 1) ? src >> 8 : src;
          ae[pp] = and_or(d, 0x000F000Fu, c64);
          ao[pp] = and_or(d, 0x00F000F0u, c54);
          asm volatile("" : "+v"(ae[pp]), "+v"(ao[pp]));
        }
        if (q == SA + SP * pp + 1) {
          se[pp] = as_u32(as_h2(ae[pp]) - as_h2(zE));
          so[pp] = as_u32(as_h2(ao[pp]) - as_h2(zO));
          asm volatile("" : "+v"(se[pp]), "+v"(so[pp]));
        }
        if (q == SA + SP * pp + 2) {
          e[pp] = as_u32(as_h2(se[pp]) * as_h2(sE));
          o[pp] = as_u32(as_h2(so[pp]) * as_h2(sO));
          asm volatile("" : "+v"(e[pp]), "+v"(o[pp]));
        }
      }
      body(q);
      __builtin_amdgcn_sched_barrier(0);
    }
    wf[cur ^ 1][0] = __builtin_bit_cast(h8, e);
    wf[cur ^ 1][1] = __builtin_bit_cast(h8, o);
  };

  auto step = [&](int kt, auto stc) __attribute__((always_inline)) {
    constexpr int ST = decltype(stc)::value;
    constexpr int NST = (ST + 1) % 3, PST = (ST + 2) % 3;
    // parts 1..3 of step kt + 2 into stage PST (free since step kt - 1's barrier)
    auto part = [&](int j) __attribute__((always_inline)) {
      return [&, j](int q) __attribute__((always_inline)) {
        if (q % DMA_GAP == 0 && q / DMA_GAP < PB) issue_one(kt + 2, PST, PA + (j - 1) * PB + q / DMA_GAP);
      };
    };
    slice(0, ST, 1, part(1));
    slice(1, ST, 2, part(2));
    slice(0, ST, 3, part(3));
    __builtin_amdgcn_s_waitcnt(WAIT_BAR);
    barrier();
    load_scales(NST);
    // part 0 of step kt + 3 into stage ST (free from this barrier on)
    slice(1, NST, 0, [&](int q) {
      if (q % DMA_GAP == 0 && q / DMA_GAP < PA) issue_one(kt + 3, ST, q / DMA_GAP);
    });
  };
  int kt = 0;
  for (; kt + 2 < nk; kt += 3) {
    step(kt, std::integral_constant<int, 0>{});
    step(kt + 1, std::integral_constant<int, 1>{});
    step(kt + 2, std::integral_constant<int, 2>{});
  }
  if (kt < nk) step(kt, std::integral_constant<int, 0>{});
  if (kt + 1 < nk) step(kt + 1, std::integral_constant<int, 1>{});
  __builtin_amdgcn_s_waitcnt(0);

  // Epilogue: element 4g + e of accumulator (mb, nb) is row 32 (MB wm + mb) + j,
  // column 64 wn + 16 g + 8 h + 2 e + nb of the tile.
  if (MODE == T_GATE_UP) {
    // g = 0, 1: gate of activation columns a0 + 32 wn + 16 g + 8 h + 2 e + nb;
    // g + 2: up of the same columns
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int m = tile.m0 + 32 * (MB * wm + mb) + j;
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int acol = a0 + 32 * wn + 16 * g + 8 * h;
        u32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          _Float16 r[2];
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) {
            const float gv = (float)(_Float16)acc[mb][nb][4 * g + e];
            const float uv = (float)(_Float16)acc[mb][nb][4 * (g + 2) + e];
            float sg = 1.0f + expf(-gv);
            asm volatile("" : "+v"(sg));
            r[nb] = h_of_rounded(gv / sg * uv);
          }
          v[e] = as_u32(f16x2{r[0], r[1]});
        }
        if (m < M && acol < I) *reinterpret_cast<u32x4*>(Y + (int64_t)m * I + acol) = v;
      }
    }
    return;
  }
  if constexpr (MODE == T_PLAIN) {
    // The tile goes through LDS so that the stores write whole rows: a
    // wavefront's 16-byte store instruction covers 2 rows x 512 bytes instead
    // of 32 bytes of each of 32 rows.  Every wavefront has finished reading
    // the stages (the DMAs past the last step were waited for above).
    constexpr int TN = 64 * WN;  // tile columns
    __syncthreads();
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    lds_u8* const cbase = (lds_u8*)(__attribute__((address_space(3))) void*)lds;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int r = 32 * (MB * wm + mb) + j;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = as_u32(f16x2{(_Float16)acc[mb][0][4 * g + e], (_Float16)acc[mb][1][4 * g + e]});
        // columns 64 wn + 16 g + 8 h .. +7 of row r
        *(__attribute__((address_space(3))) u32x4*)(cbase + (r * C_STRIDE + 64 * wn + 16 * g + 8 * h) * 2) = v;
      }
    }
    __syncthreads();  // the LDS writes of every wavefront have landed
    const int rows = min(TM, M - tile.m0), cols = min(TN, N - tile.n0);
    constexpr int CPR = TN / 8;  // 16-byte chunks per row
#pragma unroll 4
    for (int idx = t; idx < TM * CPR; idx += 256) {
      const int r = idx / CPR, ch = idx % CPR;
      const u32x4 v = *(__attribute__((address_space(3))) const u32x4*)(cbase + (r * C_STRIDE + ch * 8) * 2);
      if (r < rows && ch * 8 < cols) *reinterpret_cast<u32x4*>(Y + (int64_t)(tile.m0 + r) * N + tile.n0 + ch * 8) = v;
    }
    return;
  }
  const int col0 = tile.n0 + 64 * wn + 8 * h;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = tile.m0 + 32 * (MB * wm + mb) + j;
    int64_t dst = m;
    float rw = 1.f;
    if (MODE == T_DOWN) {
      dst = row_pid[mb];
      rw = row_w[mb];
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = col0 + 16 * g;
      u32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (MODE == T_DOWN)
          v[e] = as_u32(f16x2{h_of_rounded(acc[mb][0][4 * g + e] * rw), h_of_rounded(acc[mb][1][4 * g + e] * rw)});
        else
          v[e] = as_u32(f16x2{(_Float16)acc[mb][0][4 * g + e], (_Float16)acc[mb][1][4 * g + e]});
      }
      const bool ok = MODE == T_DOWN ? (unsigned)dst < (unsigned)rm.pairs : m < M;
      if (ok && n < N) *reinterpret_cast<u32x4*>(Y + dst * N + n) = v;
    }
  }
}
}  // namespace p8

// Blocks [0, n_full) take 256-row tiles of columns [0, 256 n_split); blocks
// n_full .. take 192-row tiles of the remaining columns.  Each part is
// numbered XCD-aware on its own (both start at a multiple of 8 blocks).
__global__ void __launch_bounds__(256, 1)
    w4a16_prefill(const _Float16* __restrict__ A, const uint8_t* __restrict__ W, const _Float16* __restrict__ S,
                   const uint8_t* __restrict__ Z, _Float16* __restrict__ Y, int M, int N, int K, int group,
                   int tiles_m, int n_split, int n_full, int tail_m, int tail_n, int tail_blocks) {
  extern __shared__ __attribute__((aligned(16))) _Float16 lds_h[];
  uint8_t* const lds = reinterpret_cast<uint8_t*>(lds_h);
  const int b = blockIdx.x;
  if (b < n_full) {
    p8::tile4<8>(lds, A, W, S, Z, Y, M, N, K, group, p8::tile_of(b, n_full, tiles_m, n_split, 256, 0));
  } else {
    const int tb = b - n_full;
    const int n_tail = tail_m * tail_n;
    const int idx = p8::remap_xcd(tb, tail_blocks);
    if (idx >= n_tail) return;
    p8::tile4<6>(lds, A, W, S, Z, Y, M, N, K, group, p8::tile_in_grid(idx, tail_m, tail_n, 192, n_split * BN));
  }
}

// Grouped (MoE) variant: rows offsets[e] .. offsets[e+1] of A use expert e's
// weights.  The grid is an upper bound (sum over experts of ceil(rows / 256)
// <= R / 256 + E tile rows, times the N tiles); each block walks the E + 1
// offsets to find its expert and tile row, and blocks past the last tile exit.
// Tile ids are regrouped per XCD as in the dense kernel, so the blocks
// resident on one XCD work on neighbouring tiles of the same expert.  A tile
// is the dense kernel's 256 x 256 tile on the expert's operands, its A and Y
// based at the tile's first row with the rows up to the expert's last as the
// valid ones, so each expert segment equals the dense product bit for bit.
__global__ void __launch_bounds__(256, 1)
    w4a16_grouped(const _Float16* __restrict__ A, const uint8_t* __restrict__ W, const _Float16* __restrict__ S,
                  const uint8_t* __restrict__ Z, const int* __restrict__ offsets, _Float16* __restrict__ Y, int R,
                  int experts, int N, int K, int group, int tiles_n) {
  extern __shared__ __attribute__((aligned(16))) _Float16 lds_h[];
  uint8_t* const lds = reinterpret_cast<uint8_t*>(lds_h);
  const int bid = grouped_block_id();
  const int mt = bid / tiles_n, nt = bid - mt * tiles_n;
  int e = 0, m0 = 0, m_end = 0;
  if (!grouped_tile(offsets, experts, R, mt, e, m0, m_end)) return;  // beyond the last tile: uniform
  const int64_t wstride = (int64_t)K * (N / 2), sstride = (int64_t)(K / group) * N, zstride = (int64_t)(K / group) * (N / 2);
  // a last column tile of at most 128 columns (N = 1408 is 5.5 tiles) runs
  // as 256 x 128: half the MFMAs, the same dequantisation per wavefront
  if (N - nt * BN <= BN / 2)
    p8::tile4<4, 2>(lds, A + (int64_t)m0 * K, W + e * wstride, S + e * sstride, Z + e * zstride,
                    Y + (int64_t)m0 * N, m_end - m0, N, K, group, Tile{0, nt * BN});
  else
    p8::tile4<8>(lds, A + (int64_t)m0 * K, W + e * wstride, S + e * sstride, Z + e * zstride, Y + (int64_t)m0 * N,
                 m_end - m0, N, K, group, Tile{0, nt * BN});
}

// MoE gate/up projection: rows of the pair space (sorted by expert, offsets[e]
// .. offsets[e+1] for expert e) gather their token's activation row X[ids[m] /
// topk], multiply by expert e's W13 [K, 2I] and write fp16(silu(gate) * up),
// I columns per row, in the same sorted row order.  128 activation columns per
// tile (64 for a last tile of at most 64: the 256 x 128 layout).
__global__ void __launch_bounds__(256, 1)
    moe_gate_up(const _Float16* __restrict__ X, const int* __restrict__ ids, const int* __restrict__ offsets,
                const uint8_t* __restrict__ W, const _Float16* __restrict__ S, const uint8_t* __restrict__ Z,
                _Float16* __restrict__ act, int tokens, int topk, int pairs, int experts, int I, int K, int group,
                int tiles_n) {
  extern __shared__ __attribute__((aligned(16))) _Float16 lds_h[];
  uint8_t* const lds = reinterpret_cast<uint8_t*>(lds_h);
  const int bid = grouped_block_id();
  const int mt = bid / tiles_n, nt = bid - mt * tiles_n;
  int e = 0, m0 = 0, m_end = 0;
  if (!grouped_tile(offsets, experts, pairs, mt, e, m0, m_end)) return;
  const int N = 2 * I;
  const int64_t wstride = (int64_t)K * I, sstride = (int64_t)(K / group) * N, zstride = (int64_t)(K / group) * I;
  RowMap rm;
  rm.ids = ids + m0;
  rm.topk = topk;
  rm.pairs = pairs;
  if (I - nt * (BN / 2) <= BN / 4)
    p8::tile4<4, 2, p8::T_GATE_UP>(lds, X, W + e * wstride, S + e * sstride, Z + e * zstride, act + (int64_t)m0 * I,
                                   m_end - m0, N, K, group, Tile{0, nt * BN}, tokens, rm);
  else
    p8::tile4<8, 4, p8::T_GATE_UP>(lds, X, W + e * wstride, S + e * sstride, Z + e * zstride, act + (int64_t)m0 * I,
                                   m_end - m0, N, K, group, Tile{0, nt * BN}, tokens, rm);
}

// MoE down projection: sorted activation rows times expert e's W2 [I, H]; row m
// is scaled by its pair's routing weight w[ids[m]] in fp32 and stored, as fp16,
// at row ids[m] of Y [pairs, H] (token-major: pair t * topk + j).
__global__ void __launch_bounds__(p8::THREADS, 1)
    moe_down(const _Float16* __restrict__ act, const int* __restrict__ ids, const int* __restrict__ offsets,
             const float* __restrict__ w, const uint8_t* __restrict__ W, const _Float16* __restrict__ S,
             const uint8_t* __restrict__ Z, _Float16* __restrict__ Y, int pairs, int experts, int H, int I,
             int group, int tiles_n) {
  extern __shared__ __attribute__((aligned(16))) _Float16 lds_h[];
  uint8_t* const lds = reinterpret_cast<uint8_t*>(lds_h);
  const int bid = grouped_block_id();
  const int mt = bid / tiles_n, nt = bid - mt * tiles_n;
  int e = 0, m0 = 0, m_end = 0;
  if (!grouped_tile(offsets, experts, pairs, mt, e, m0, m_end)) return;
  const int64_t wstride = (int64_t)I * (H / 2), sstride = (int64_t)(I / group) * H, zstride = (int64_t)(I / group) * (H / 2);
  RowMap rm;
  rm.ids = ids + m0;
  rm.w = w;
  rm.pairs = pairs;
  if (H - nt * BN <= BN / 2)
    p8::tile8<2, 2, p8::T_DOWN>(lds, act + (int64_t)m0 * I, W + e * wstride, S + e * sstride, Z + e * zstride, Y,
                                m_end - m0, H, I, group, Tile{0, nt * BN}, m_end - m0, rm);
  else
    p8::tile8<4, 4, p8::T_DOWN>(lds, act + (int64_t)m0 * I, W + e * wstride, S + e * sstride, Z + e * zstride, Y,
                                m_end - m0, H, I, group, Tile{0, nt * BN}, m_end - m0, rm);
}

}  // namespace w4a16
}  // namespace tb

extern "C" tb_status tb_w4a16_workspace_size(int64_t M, int64_t N, int64_t K, int64_t group, int64_t* bytes) {
  using namespace tb::w4a16;
  TB_CHECK_ARG(bytes != nullptr, "tb_w4a16_workspace_size: null output");
  TB_CHECK_ARG(M > 0 && N > 0 && K > 0 && group > 0, "tb_w4a16_workspace_size: sizes must be positive");
  *bytes = 0;
  if (M <= 16 && K % DEC_UNIT == 0) {
    const int64_t slabs = (N + DEC_COLS - 1) / DEC_COLS;
    const int splits = decode_splits((int)N, (int)K);
    if (splits > 1) *bytes = DEC_COUNTER_BYTES + (int64_t)splits * M * N * 4;
  }
  return TB_OK;
}

namespace tb {
namespace w4a16 {

// Shape and alignment checks of the dense W4A16 GEMM, shared by both entry
// points (`fn` names the caller in the messages).
static tb_status check_dense_args(const char* fn, const uint16_t* A, const uint8_t* W, const uint16_t* scales,
                                  const uint8_t* zeros, const uint16_t* Y, int64_t M, int64_t N, int64_t K,
                                  int64_t group) {
  TB_CHECK_ARG(A && W && scales && zeros && Y, "%s: null pointer", fn);
  TB_CHECK_ARG(M > 0 && N > 0 && K > 0 && group > 0, "%s: sizes must be positive", fn);
  TB_CHECK_ARG(M < (1 << 30) && N < (1 << 30) && K < (1 << 30), "%s: sizes too large", fn);
  TB_CHECK_ARG(N % 8 == 0, "%s: N must be a multiple of 8 (got %lld)", fn, (long long)N);
  TB_CHECK_ARG(K % BK == 0 && group % BK == 0 && K % group == 0,
               "%s: need K %% 64 == 0, group %% 64 == 0 and K %% group == 0 (K=%lld group=%lld)", fn, (long long)K,
               (long long)group);
  // Both kernels address A, W, scales and zeros through 32-bit buffer offsets
  // whose out-of-range sentinel is 2^31: every operand must stay below 2 GiB.
  TB_CHECK_ARG(M * K * 2 < (1ll << 31) && K * (N / 2) < (1ll << 31) && (K / group) * N * 2 < (1ll << 31),
               "%s: A, W and scales must each be smaller than 2 GiB (M=%lld N=%lld K=%lld)", fn, (long long)M,
               (long long)N, (long long)K);
  TB_CHECK_ALIGN(A, 16, "A");
  TB_CHECK_ALIGN(W, 4, "W");
  TB_CHECK_ALIGN(scales, 16, "scales");
  TB_CHECK_ALIGN(zeros, 4, "zeros");
  TB_CHECK_ALIGN(Y, 2, "Y");
  if (M <= 16) {
    const int64_t slabs = (N + DEC_COLS - 1) / DEC_COLS;
    const int splits = decode_splits((int)N, (int)K);
    TB_CHECK_ARG(splits == 1 || (slabs <= DEC_MAX_SLABS && (int64_t)splits * M * N * 4 < (1ll << 31)),
                 "%s: N=%lld is too wide for the decode kernel", fn, (long long)N);
  }
  return TB_OK;
}

// Launch of the dense W4A16 GEMM after the checks: the split-K decode kernel
// for M <= 16 (counters at `workspace`, fp32 partials DEC_COUNTER_BYTES past
// it), the MFMA prefill kernel otherwise.
// How the dense prefill covers the output (256-row tiles over the first
// n_split tile columns, 192-row tiles over the rest): tb::plan::plan_prefill,
// prefill_plan.h, a closed-form evaluation of the greedy schedule per split.
using tb::plan::PrefillPlan;
using tb::plan::plan_prefill;

static tb_status launch_dense(const char* fn, const uint16_t* A, const uint8_t* W, const uint16_t* scales,
                              const uint8_t* zeros, uint16_t* Y, int64_t M, int64_t N, int64_t K, int64_t group,
                              void* workspace, hipStream_t stream) {
  if (M <= 16) {
    const int64_t slabs = (N + DEC_COLS - 1) / DEC_COLS;
    const int splits = decode_splits((int)N, (int)K);
    int* counters = reinterpret_cast<int*>(workspace);
    float* partials =
        splits > 1 ? reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + DEC_COUNTER_BYTES) : nullptr;
    if (N % 16 == 0)
      hipLaunchKernelGGL(w4a16_decode<false>, dim3((unsigned)(slabs * splits)), dim3(DEC_THREADS), 0, stream,
                         reinterpret_cast<const _Float16*>(A), W, reinterpret_cast<const _Float16*>(scales), zeros,
                         reinterpret_cast<_Float16*>(Y), partials, counters, (int)M, (int)N, (int)K, (int)group, splits);
    else
      hipLaunchKernelGGL(w4a16_decode<true>, dim3((unsigned)(slabs * splits)), dim3(DEC_THREADS), 0, stream,
                         reinterpret_cast<const _Float16*>(A), W, reinterpret_cast<const _Float16*>(scales), zeros,
                         reinterpret_cast<_Float16*>(Y), partials, counters, (int)M, (int)N, (int)K, (int)group, splits);
    return tb::launch_status(fn);
  }
  if (tb_status st = tb::reserve_lds(reinterpret_cast<const void*>(&w4a16_prefill), p8::LDS_BYTES, fn)) return st;
  const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
  const PrefillPlan pl = plan_prefill((int)M, tiles_m, tiles_n, device_cus());
  hipLaunchKernelGGL(w4a16_prefill, dim3(pl.n_full + pl.tail_blocks), dim3(256), p8::LDS_BYTES, stream,
                     reinterpret_cast<const _Float16*>(A), W, reinterpret_cast<const _Float16*>(scales), zeros,
                     reinterpret_cast<_Float16*>(Y), (int)M, (int)N, (int)K, (int)group, tiles_m, pl.n_split,
                     pl.n_full, pl.tail_m, pl.tail_n, pl.tail_blocks);
  return tb::launch_status(fn);
}

// ---------------------------------------------------------------- no-allocation variant
// The decode's split-K counters and partials live in one file-scope device
// array per GPU instead of a caller workspace.  Its size is the decode's need
// at M <= 16 on a 256-CU device: slabs x splits never exceeds the CU count, so
// the partials hold at most 256 blocks x 16 rows x 256 columns of fp32
// (4 MiB), behind the 16 KiB of counters.
constexpr int64_t NOALLOC_SCRATCH_BYTES = DEC_COUNTER_BYTES + 256ll * 16 * DEC_COLS * 4;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

__global__ void __launch_bounds__(256) clear_counters(int* __restrict__ c, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) c[i] = 0;
}

struct ScratchSlot {
  void* ptr = nullptr;  // this device's address of `scratch`
  bool ready = false;
};
static std::mutex g_scratch_mu;
static ScratchSlot g_scratch[64];

// This device's address of `scratch`, looked up once per device (with that
// device current) by hipGetSymbolAddress: in host code the array's name is
// only a stand-in, never a device address.  The first call on a device also
// clears the counters with a kernel on the caller's stream (not hipMemset: the
// call may be under graph capture); the decode leaves them at zero afterwards.
static tb_status scratch_of_current_device(const char* fn, hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    tb::set_error("%s: no usable current device", fn);
    return TB_E_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchSlot& slot = g_scratch[dev];
  if (!slot.ready) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      tb::set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", fn, dev, hipGetErrorString(e));
      return TB_E_HIP;
    }
    const int n = (int)(DEC_COUNTER_BYTES / 4);
    hipLaunchKernelGGL(clear_counters, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       reinterpret_cast<int*>(p), n);
    if (tb_status st = tb::launch_status(fn)) return st;
    slot.ptr = p;
    slot.ready = true;
  }
  *out = slot.ptr;
  return TB_OK;
}

}  // namespace w4a16
}  // namespace tb

extern "C" tb_status tb_w4a16_gemm(const uint16_t* A, const uint8_t* W, const uint16_t* scales, const uint8_t* zeros,
                                   uint16_t* Y, int64_t M, int64_t N, int64_t K, int64_t group, void* workspace,
                                   int64_t workspace_bytes, hipStream_t stream) {
  using namespace tb::w4a16;
  const char* fn = "tb_w4a16_gemm";
  if (tb_status st = check_dense_args(fn, A, W, scales, zeros, Y, M, N, K, group)) return st;
  if (M <= 16) {
    int64_t need = 0;
    tb_w4a16_workspace_size(M, N, K, group, &need);
    if (need > 0) {
      TB_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                   "tb_w4a16_gemm: M=%lld needs a %lld-byte workspace (got %lld)", (long long)M, (long long)need,
                   (long long)workspace_bytes);
      if (!tb::aligned(workspace, 256)) {
        tb::set_error("tb_w4a16_gemm: workspace must be 256-byte aligned");
        return TB_E_ALIGN;
      }
    }
  }
  return launch_dense(fn, A, W, scales, zeros, Y, M, N, K, group, workspace, stream);
}

extern "C" tb_status tb_w4a16_gemm_noalloc(const uint16_t* A, const uint8_t* W, const uint16_t* scales,
                                           const uint8_t* zeros, uint16_t* Y, int64_t M, int64_t N, int64_t K,
                                           int64_t group, hipStream_t stream) {
  using namespace tb::w4a16;
  const char* fn = "tb_w4a16_gemm_noalloc";
  if (tb_status st = check_dense_args(fn, A, W, scales, zeros, Y, M, N, K, group)) return st;
  void* ws = nullptr;
  if (M <= 16) {
    int64_t need = 0;
    tb_w4a16_workspace_size(M, N, K, group, &need);
    TB_CHECK_ARG(need <= NOALLOC_SCRATCH_BYTES,
                 "tb_w4a16_gemm_noalloc: M=%lld N=%lld needs %lld bytes of split-K scratch, the static scratch "
                 "holds %lld (use tb_w4a16_gemm with a workspace)",
                 (long long)M, (long long)N, (long long)need, (long long)NOALLOC_SCRATCH_BYTES);
    if (need > 0)
      if (tb_status st = scratch_of_current_device(fn, stream, &ws)) return st;
  }
  return launch_dense(fn, A, W, scales, zeros, Y, M, N, K, group, ws, stream);
}

extern "C" tb_status tb_moe_w4a16_grouped_gemm(const uint16_t* A, const uint8_t* W, const uint16_t* scales,
                                               const uint8_t* zeros, const int32_t* offsets, uint16_t* Y, int64_t R,
                                               int64_t experts, int64_t N, int64_t K, int64_t group,
                                               hipStream_t stream) {
  using namespace tb::w4a16;
  TB_CHECK_ARG(A && W && scales && zeros && offsets && Y, "tb_moe_w4a16_grouped_gemm: null pointer");
  TB_CHECK_ARG(R > 0 && experts > 0 && N > 0 && K > 0 && group > 0, "tb_moe_w4a16_grouped_gemm: sizes must be positive");
  TB_CHECK_ARG(experts <= 4096, "tb_moe_w4a16_grouped_gemm: at most 4096 experts (got %lld)", (long long)experts);
  TB_CHECK_ARG(N % 8 == 0, "tb_moe_w4a16_grouped_gemm: N must be a multiple of 8 (got %lld)", (long long)N);
  TB_CHECK_ARG(K % BK == 0 && group % BK == 0 && K % group == 0,
               "tb_moe_w4a16_grouped_gemm: need K %% 64 == 0, group %% 64 == 0 and K %% group == 0");
  TB_CHECK_ARG(R * K * 2 < (1ll << 31) * 2 - 1, "tb_moe_w4a16_grouped_gemm: A must be smaller than 4 GiB");
  TB_CHECK_ARG(K * (N / 2) < (1ll << 31), "tb_moe_w4a16_grouped_gemm: one expert's weights must be < 2 GiB");
  TB_CHECK_ALIGN(A, 16, "A");
  TB_CHECK_ALIGN(W, 4, "W");
  TB_CHECK_ALIGN(scales, 16, "scales");
  TB_CHECK_ALIGN(zeros, 4, "zeros");
  TB_CHECK_ALIGN(Y, 16, "Y");
  if (tb_status st = tb::reserve_lds(reinterpret_cast<const void*>(&w4a16_grouped), p8::LDS_BYTES, "tb_moe_w4a16_grouped_gemm")) return st;
  const int64_t tiles_n = (N + BN - 1) / BN;
  const int64_t tile_rows = (R + BM - 1) / BM + experts;  // upper bound on sum_e ceil(rows_e / 256)
  const int64_t blocks = tile_rows * tiles_n;
  TB_CHECK_ARG(blocks < (1ll << 31), "tb_moe_w4a16_grouped_gemm: problem too large");
  hipLaunchKernelGGL(w4a16_grouped, dim3((unsigned)blocks), dim3(256), p8::LDS_BYTES, stream,
                     reinterpret_cast<const _Float16*>(A), W, reinterpret_cast<const _Float16*>(scales), zeros, offsets,
                     reinterpret_cast<_Float16*>(Y), (int)R, (int)experts, (int)N, (int)K, (int)group, (int)tiles_n);
  return tb::launch_status("tb_moe_w4a16_grouped_gemm");
}


extern "C" tb_status tb_moe_w4a16_gate_up(const uint16_t* X, const int32_t* sorted_ids, const int32_t* offsets,
                                          const uint8_t* W13, const uint16_t* S13, const uint8_t* Z13, uint16_t* act,
                                          int64_t tokens, int64_t topk, int64_t experts, int64_t H, int64_t I,
                                          int64_t group, hipStream_t stream) {
  using namespace tb::w4a16;
  const char* fn = "tb_moe_w4a16_gate_up";
  TB_CHECK_ARG(X && sorted_ids && offsets && W13 && S13 && Z13 && act, "%s: null pointer", fn);
  TB_CHECK_ARG(tokens > 0 && topk > 0 && experts > 0 && H > 0 && I > 0 && group > 0, "%s: sizes must be positive", fn);
  TB_CHECK_ARG(experts <= 4096 && topk <= experts, "%s: need topk <= experts <= 4096", fn);
  const int64_t pairs = tokens * topk;
  TB_CHECK_ARG(pairs < (1ll << 31), "%s: tokens * topk must be < 2^31", fn);
  TB_CHECK_ARG(I % 8 == 0, "%s: I must be a multiple of 8 (got %lld)", fn, (long long)I);
  TB_CHECK_ARG(H % BK == 0 && group % BK == 0 && H % group == 0,
               "%s: need H %% 64 == 0, group %% 64 == 0 and H %% group == 0 (H=%lld group=%lld)", fn, (long long)H,
               (long long)group);
  TB_CHECK_ARG(tokens * H * 2 < (1ll << 32) && H * I < (1ll << 31) && pairs * I * 2 < (1ll << 62),
               "%s: X must be < 4 GiB and one expert's W13 < 2 GiB", fn);
  TB_CHECK_ALIGN(X, 16, "X");
  TB_CHECK_ALIGN(W13, 4, "W13");
  TB_CHECK_ALIGN(S13, 16, "S13");
  TB_CHECK_ALIGN(Z13, 4, "Z13");
  TB_CHECK_ALIGN(act, 16, "act");
  if (tb_status st = tb::reserve_lds(reinterpret_cast<const void*>(&moe_gate_up), p8::LDS_BYTES, fn)) return st;
  const int64_t tiles_n = (I + BN / 2 - 1) / (BN / 2);
  const int64_t tile_rows = (pairs + BM - 1) / BM + experts;
  const int64_t blocks = tile_rows * tiles_n;
  TB_CHECK_ARG(blocks < (1ll << 31), "%s: problem too large", fn);
  hipLaunchKernelGGL(moe_gate_up, dim3((unsigned)blocks), dim3(256), p8::LDS_BYTES, stream,
                     reinterpret_cast<const _Float16*>(X), sorted_ids, offsets, W13,
                     reinterpret_cast<const _Float16*>(S13), Z13, reinterpret_cast<_Float16*>(act), (int)tokens,
                     (int)topk, (int)pairs, (int)experts, (int)I, (int)H, (int)group, (int)tiles_n);
  return tb::launch_status(fn);
}

extern "C" tb_status tb_moe_w4a16_down(const uint16_t* act, const int32_t* sorted_ids, const int32_t* offsets,
                                       const float* topk_weights, const uint8_t* W2, const uint16_t* S2,
                                       const uint8_t* Z2, uint16_t* Y, int64_t pairs, int64_t experts, int64_t I,
                                       int64_t H, int64_t group, hipStream_t stream) {
  using namespace tb::w4a16;
  const char* fn = "tb_moe_w4a16_down";
  TB_CHECK_ARG(act && sorted_ids && offsets && topk_weights && W2 && S2 && Z2 && Y, "%s: null pointer", fn);
  TB_CHECK_ARG(pairs > 0 && experts > 0 && H > 0 && I > 0 && group > 0, "%s: sizes must be positive", fn);
  TB_CHECK_ARG(experts <= 4096 && pairs < (1ll << 31), "%s: need experts <= 4096 and pairs < 2^31", fn);
  TB_CHECK_ARG(H % 8 == 0, "%s: H must be a multiple of 8 (got %lld)", fn, (long long)H);
  TB_CHECK_ARG(I % BK == 0 && group % BK == 0 && I % group == 0,
               "%s: need I %% 64 == 0, group %% 64 == 0 and I %% group == 0 (I=%lld group=%lld)", fn, (long long)I,
               (long long)group);
  TB_CHECK_ARG(pairs * I * 2 < (1ll << 32) && I * (H / 2) < (1ll << 31),
               "%s: act must be < 4 GiB and one expert's W2 < 2 GiB", fn);
  TB_CHECK_ALIGN(act, 16, "act");
  TB_CHECK_ALIGN(W2, 4, "W2");
  TB_CHECK_ALIGN(S2, 16, "S2");
  TB_CHECK_ALIGN(Z2, 4, "Z2");
  TB_CHECK_ALIGN(Y, 16, "Y");
  if (tb_status st = tb::reserve_lds(reinterpret_cast<const void*>(&moe_down), p8::LDS_BYTES, fn)) return st;
  const int64_t tiles_n = (H + BN - 1) / BN;
  const int64_t tile_rows = (pairs + BM - 1) / BM + experts;
  const int64_t blocks = tile_rows * tiles_n;
  TB_CHECK_ARG(blocks < (1ll << 31), "%s: problem too large", fn);
  hipLaunchKernelGGL(moe_down, dim3((unsigned)blocks), dim3(p8::THREADS), p8::LDS_BYTES, stream,
                     reinterpret_cast<const _Float16*>(act), sorted_ids, offsets, topk_weights, W2,
                     reinterpret_cast<const _Float16*>(S2), Z2, reinterpret_cast<_Float16*>(Y), (int)pairs,
                     (int)experts, (int)H, (int)I, (int)group, (int)tiles_n);
  return tb::launch_status(fn);
}
