// The reference's plain GEMM operators on the CDNA4 matrix cores:
//
//   matmul_int8            out int32 [M, N] = A int8 [M, K] @ unpack(B) with B
//                          holding four 2-bit fields per byte (value - 1),
//                          field i of row kb being row i * K/4 + kb of B;
//   matmul_fp32_fp16_fp8   fp16: Y = fp16(A @ B), fp32 accumulation;
//                          fp8 (e4m3): Y = e4m3(bf16(A @ B)), the reference's
//                          unit-scale _scaled_mm to bf16 followed by its cast;
//                          fp32: A @ B from three bf16 products per term (see
//                          below), fp32 accumulation and output.
//
// All four are one "NT" kernel: both operands K-contiguous, A as [M, K] and
// the second operand transposed to [N, K], 128 bytes of K per step.  A
// preparation pass writes that transposed operand into the caller's workspace
// (a tiled LDS transpose; for int8 it also unpacks the 2-bit fields, for fp32
// it splits the values).  The GEMM kernel is the fp8 GEMM's design: operands
// stream HBM -> LDS through the buffer unit (buffer_load ... lds) one step
// ahead into two stages, rows in 16-byte chunks with chunk c of row r at slot
// c ^ ((r ^ (r >> 3)) & 7) (conflict-free DMA writes and fragment reads).
// The MFMA takes the B^T fragment as its first operand, so each lane ends with
// four consecutive output columns per accumulator group and stores them
// straight from registers.  Two tile shapes: 256 x 256 on eight wavefronts
// (128 x 64 each) and 128 x 128 on four (64 x 64 each) for grids too small for
// 256 x 256 tiles.  matmul_int8 at M = N = 2048 (64 tiles of 256 x 256) splits
// K instead when K is deep: 128 x 128 int8 tiles need 32 KiB of operands per
// CU per 128-byte K step, about the L2-to-CU bandwidth at the MFMA rate, where
// 256 x 256 tiles need half that per MAC; each split writes an int32 partial
// plane and a pass adds the planes (exact, so the split does not change a bit).
//
// fp32 without an fp32-rate penalty: x = hi + lo with hi = bf16(x) and
// lo = bf16(x - hi) (x - hi is exact in fp32), and
//   A @ B ~= A_hi @ B_hi + A_hi @ B_lo + A_lo @ B_hi,
// dropping A_lo @ B_lo (relative size 2^-16).  That is one bf16 GEMM over
// K' = 3K of A' = [A_hi | A_hi | A_lo] and B'^T = [B_hi^T | B_lo^T | B_hi^T],
// accurate to about 2^-16 per product: finer than the TF32 the reference
// allows for its fp32 matmul (10 mantissa bits) and run at the bf16 rate.
#include "tb_common.h"

#include <algorithm>

namespace tb {
namespace ntg {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

enum Kind { KIND_FP8 = 0, KIND_F16 = 1, KIND_BF16 = 2, KIND_I8 = 3 };
enum Out { OUT_BF16 = 0, OUT_E4M3 = 1, OUT_F16 = 2, OUT_F32 = 3, OUT_I32 = 4 };

constexpr int BK = 128;  // bytes of K per step
constexpr uint32_t RSRC_DW3 = 0x00020000u;
constexpr uint32_t OOB = 0x80000000u;

__device__ __forceinline__ int slot(int row, int chunk) { return row * BK + ((chunk ^ ((row ^ (row >> 3)) & 7)) << 4); }

__device__ __forceinline__ i32x4 make_rsrc4(const void* p, uint32_t bytes) {
  const uint64_t base = (uint64_t)(uintptr_t)p;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)base);
  r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32) & 0xFFFF);
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = (int)RSRC_DW3;
  return r;
}

// One 16-byte-per-lane DMA into LDS (wave-uniform base, lane l -> +16 l), as
// inline asm so the compiler does not tie barriers to its completion; the
// kernel waits for it explicitly (vmcnt) before the barrier that publishes it.
__device__ __forceinline__ void dma16(uint32_t lds_addr, uint32_t voff, const i32x4& rsrc, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane((int)lds_addr)), "v"(voff), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane((int)soff))
               : "memory", "m0");
}

template <int BM, int BN>
__device__ __forceinline__ void tile_of_block(int bid, int tiles_m, int tiles_n, int& m0, int& n0) {
  constexpr int GROUP_M = 8;
  const int nb = tiles_m * tiles_n;
  if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);  // contiguous run of tiles per XCD
  const int per_group = GROUP_M * tiles_n;
  const int group = bid / per_group;
  const int first_m = group * GROUP_M;
  const int rows = min(tiles_m - first_m, GROUP_M);
  const int in_group = bid - group * per_group;
  m0 = (first_m + in_group % rows) * BM;
  n0 = (in_group / rows) * BN;
}

template <int KIND>
struct Acc {
  typedef f32x16 type;
};
template <>
struct Acc<KIND_I8> {
  typedef i32x16 type;
};

// One MFMA step of 32 bytes of K (64 for fp8) on 16 (32) bytes per lane.
template <int KIND>
__device__ __forceinline__ typename Acc<KIND>::type mfma(const i32x8& b, const i32x8& a, typename Acc<KIND>::type c) {
  if constexpr (KIND == KIND_FP8) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, 0, 0, 0);
  } else {
    const i32x4 b4 = {b[0], b[1], b[2], b[3]}, a4 = {a[0], a[1], a[2], a[3]};
    if constexpr (KIND == KIND_F16)
      return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8, b4), __builtin_bit_cast(h8, a4), c, 0, 0, 0);
    else if constexpr (KIND == KIND_BF16)
      return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf8, b4), __builtin_bit_cast(bf8, a4), c, 0, 0,
                                                     0);
    else
      return __builtin_amdgcn_mfma_i32_32x32x32_i8(b4, a4, c, 0, 0, 0);
  }
}

template <int KIND, int OUT, int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64, 1)
    nt_gemm(const uint8_t* __restrict__ A, const uint8_t* __restrict__ BT, void* __restrict__ Yv,
            const float* __restrict__ sa, const float* __restrict__ sw, int M, int N, int Kb, int tiles_m,
            int tiles_n, int splits) {
  constexpr int WAVES = (BM / WM) * (BN / WN), THREADS = WAVES * 64;
  constexpr int FI = WM / 32, FJ = WN / 32;
  constexpr int A_STAGE = BM * BK, B_STAGE = BN * BK;
  constexpr int A_DMA = BM / 8 / WAVES, B_DMA = BN / 8 / WAVES;  // 1 KiB DMA instructions per wave and step
  constexpr int SUB = KIND == KIND_FP8 ? 2 : 4;                    // MFMA k-substeps per step
  static_assert(A_DMA * WAVES * 8 == BM && B_DMA * WAVES * 8 == BN, "tile rows must split evenly over the DMA");
  typedef typename Acc<KIND>::type acc_t;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  // Split-K (int32 output only): block b computes K steps [split * nk / splits,
  // (split + 1) * nk / splits), split = b / tiles, of tile b % tiles into
  // partial plane `split` of Yv (each plane M x N); a reduction pass adds the
  // planes (int32 sums are exact in any order, so the result equals the
  // unsplit product bit for bit).  Each split's blocks are consecutive, so the
  // per-XCD tile grouping below sees the same block ids as without splits.
  // With splits dividing the 8 XCDs (blocks go round-robin over them), split
  // s runs on XCDs s*G .. s*G+G-1 (G = 8 / splits) and each of those takes a
  // contiguous run of tile columns, so an XCD's L2 holds its K range of every
  // A row panel once and of its own B column panels only.
  const int tiles = tiles_m * tiles_n;
  int split, m0, n0;
  if (splits > 1 && 8 % splits == 0 && tiles % (8 / splits) == 0) {
    const int G = 8 / splits, xcd = (int)blockIdx.x & 7, j = (int)blockIdx.x >> 3;
    split = xcd / G;
    const int t = (xcd % G) * (tiles / G) + j;  // column-major over the split's tiles
    m0 = (t % tiles_m) * BM;
    n0 = (t / tiles_m) * BN;
  } else {
    split = (int)blockIdx.x / tiles;
    tile_of_block<BM, BN>((int)blockIdx.x % tiles, tiles_m, tiles_n, m0, n0);
  }
  if constexpr (OUT == OUT_I32) Yv = reinterpret_cast<int32_t*>(Yv) + (int64_t)split * M * N;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave / (BN / WN), wn = wave % (BN / WN);

  const i32x4 ra = make_rsrc4(A, (uint32_t)M * (uint32_t)Kb);
  const i32x4 rb = make_rsrc4(BT, (uint32_t)N * (uint32_t)Kb);
  uint32_t a_off[A_DMA], b_off[B_DMA];
  {
    const int lr = lane >> 3;
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) {
      const int row = (wave * A_DMA + i) * 8 + lr;
      const int lc = (lane & 7) ^ ((row ^ (row >> 3)) & 7);
      a_off[i] = m0 + row < M ? (uint32_t)(m0 + row) * (uint32_t)Kb + (uint32_t)lc * 16u : OOB;
    }
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) {
      const int row = (wave * B_DMA + i) * 8 + lr;
      const int lc = (lane & 7) ^ ((row ^ (row >> 3)) & 7);
      b_off[i] = n0 + row < N ? (uint32_t)(n0 + row) * (uint32_t)Kb + (uint32_t)lc * 16u : OOB;
    }
  }
  const uint32_t lds0 = (uint32_t)__builtin_amdgcn_readfirstlane(
      (int)(uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  int k_first = 0;  // first K step of this block (stage parity counts from it)
  auto issue = [&](int kt) {
    const uint32_t st = lds0 + (uint32_t)(((kt - k_first) & 1) * (A_STAGE + B_STAGE));
    const uint32_t soff = (uint32_t)(kt * BK);
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) dma16(st + (uint32_t)((wave * A_DMA + i) * 1024), a_off[i], ra, soff);
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) dma16(st + A_STAGE + (uint32_t)((wave * B_DMA + i) * 1024), b_off[i], rb, soff);
  };

  const int a_row = wm * WM + (lane & 31);
  const int b_row = wn * WN + (lane & 31);
  // fragment of substep s: fp8 reads chunks 4s + 2h and 4s + 2h + 1 (32 bytes),
  // the others chunk 2s + h (16 bytes), h = lane / 32
  auto frag = [&](const uint8_t* base, int row, int s) -> i32x8 {
    i32x8 r = {};
    if constexpr (KIND == KIND_FP8) {
      const int c0 = 4 * s + 2 * (lane >> 5);
      const i32x4 lo = *reinterpret_cast<const i32x4*>(base + slot(row, c0));
      const i32x4 hi = *reinterpret_cast<const i32x4*>(base + slot(row, c0 + 1));
      r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
      r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
    } else {
      const i32x4 v = *reinterpret_cast<const i32x4*>(base + slot(row, 2 * s + (lane >> 5)));
      r[0] = v[0]; r[1] = v[1]; r[2] = v[2]; r[3] = v[3];
    }
    return r;
  };

  acc_t acc[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j) acc[i][j] = acc_t{};

  constexpr int WAIT_VM0 = 0 | (7 << 4) | (15 << 8);
  const int nk_all = Kb / BK;
  const int k_begin = (int)((int64_t)nk_all * split / splits), k_end = (int)((int64_t)nk_all * (split + 1) / splits);
  k_first = k_begin;
  issue(k_begin);
  __builtin_amdgcn_s_waitcnt(WAIT_VM0);
  __syncthreads();
  for (int kt = k_begin; kt < k_end; ++kt) {
    const bool more = kt + 1 < k_end;
    if (more) issue(kt + 1);
    const uint8_t* sa_ = lds + ((kt - k_begin) & 1) * (A_STAGE + B_STAGE);
    const uint8_t* sb_ = sa_ + A_STAGE;
    if constexpr (KIND == KIND_FP8) {
      // Both k64 substeps' fragments are read up front; the scheduling hints
      // interleave the second substep's reads with the first substep's MFMAs.
      i32x8 fa0[FI], fb0[FJ], fa1[FI], fb1[FJ];
#pragma unroll
      for (int i = 0; i < FI; ++i) fa0[i] = frag(sa_, a_row + i * 32, 0);
#pragma unroll
      for (int j = 0; j < FJ; ++j) fb0[j] = frag(sb_, b_row + j * 32, 0);
#pragma unroll
      for (int i = 0; i < FI; ++i) fa1[i] = frag(sa_, a_row + i * 32, 1);
#pragma unroll
      for (int j = 0; j < FJ; ++j) fb1[j] = frag(sb_, b_row + j * 32, 1);
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j) acc[i][j] = mfma<KIND>(fb0[j], fa0[i], acc[i][j]);
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j) acc[i][j] = mfma<KIND>(fb1[j], fa1[i], acc[i][j]);
      constexpr int NR = 2 * (FI + FJ);  // ds_read_b128 per substep
      __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
#pragma unroll
      for (int q = 0; q < NR / 2; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * FI * FJ - NR / 2, 0);
    } else {
    // The fragments of substep s + 1 are read while the MFMAs of substep s run.
    i32x8 fa[2][FI], fb[2][FJ];
#pragma unroll
    for (int i = 0; i < FI; ++i) fa[0][i] = frag(sa_, a_row + i * 32, 0);
#pragma unroll
    for (int j = 0; j < FJ; ++j) fb[0][j] = frag(sb_, b_row + j * 32, 0);
#pragma unroll
    for (int s = 0; s < SUB; ++s) {
      const int cur = s & 1;
      if (s + 1 < SUB) {
#pragma unroll
        for (int i = 0; i < FI; ++i) fa[cur ^ 1][i] = frag(sa_, a_row + i * 32, s + 1);
#pragma unroll
        for (int j = 0; j < FJ; ++j) fb[cur ^ 1][j] = frag(sb_, b_row + j * 32, s + 1);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j) acc[i][j] = mfma<KIND>(fb[cur][j], fa[cur][i], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
    }
    }
    // stage kt + 1 must land before the barrier that hands it to the next step
    if (more) __builtin_amdgcn_s_waitcnt(WAIT_VM0);
    __syncthreads();
  }

  // Epilogue straight from registers: accumulator elements 4g .. 4g+3 of
  // fragment (i, j) are row i*32 + lane%32, columns j*32 + g*8 + (lane/32)*4 + 0..3
  // of the wave tile (N % 8 == 0, so four columns are all in or all out).
  // The fp8 scales are fetched before any branch, by buffer loads that read
  // zeros past M or N, so they are all in flight together.
  float sav[FI];
  f32x4 swv[FJ][4];
#pragma unroll
  for (int i = 0; i < FI; ++i) sav[i] = 1.f;
#pragma unroll
  for (int j = 0; j < FJ; ++j)
#pragma unroll
    for (int g = 0; g < 4; ++g) swv[j][g] = f32x4{1.f, 1.f, 1.f, 1.f};
  if constexpr (KIND == KIND_FP8) {
    if (sa) {
      const buf_rsrc_t rsa = buf_rsrc(sa, (uint32_t)M * 4u);
#pragma unroll
      for (int i = 0; i < FI; ++i) {
        const int m = m0 + a_row + i * 32;
        sav[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsa, m < M ? (uint32_t)m * 4u : BUF_OOB, 0, 0));
      }
    }
    if (sw) {
      const buf_rsrc_t rsw = buf_rsrc(sw, (uint32_t)N * 4u);
#pragma unroll
      for (int j = 0; j < FJ; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + wn * WN + j * 32 + g * 8 + (lane >> 5) * 4;
          swv[j][g] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsw, n < N ? (uint32_t)n * 4u : BUF_OOB, 0, 0));
        }
    }
  }
#pragma unroll
  for (int i = 0; i < FI; ++i) {
    const int m = m0 + a_row + i * 32;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < FJ; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * WN + j * 32 + g * 8 + (lane >> 5) * 4;
        if (n >= N) continue;
        const int64_t o = (int64_t)m * N + n;
        if constexpr (OUT == OUT_I32) {
          i32x4 v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          *reinterpret_cast<i32x4*>(reinterpret_cast<int32_t*>(Yv) + o) = v;
        } else if constexpr (OUT == OUT_F32) {
          f32x4 v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(Yv) + o) = v;
        } else if constexpr (OUT == OUT_F16) {
          u32x2 v;
          v[0] = as_u32(f16x2{(_Float16)acc[i][j][4 * g], (_Float16)acc[i][j][4 * g + 1]});
          v[1] = as_u32(f16x2{(_Float16)acc[i][j][4 * g + 2], (_Float16)acc[i][j][4 * g + 3]});
          *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(Yv) + o) = v;
        } else {
          uint32_t b[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float x = acc[i][j][4 * g + q];
            if constexpr (KIND == KIND_FP8) x = x * sav[i] * swv[j][g][q];
            b[q] = bf16_bits(x);
          }
          if constexpr (OUT == OUT_BF16) {
            u32x2 v;
            v[0] = b[0] | (b[1] << 16);
            v[1] = b[2] | (b[3] << 16);
            *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(Yv) + o) = v;
          } else {  // OUT_E4M3: the bf16 value, cast once more
            uint32_t c = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) c |= e4m3_code(__builtin_bit_cast(float, b[q] << 16)) << (8 * q);
            *reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(Yv) + o) = c;
          }
        }
      }
  }
}

// ------------------------------------------------------------------ preparation passes

// The preparation passes move 64 x 64 element tiles through LDS with 16-byte
// global loads along the source rows and 16-byte global stores along the
// destination rows (consecutive threads take consecutive chunks of one
// destination row, so each row segment is written by one coalesced group).

// B [K, N] (E = 1 or 2 bytes per element) -> B^T [N, K].  Needs N % 8 == 0 and
// K a multiple of 16 / E; partial source chunks at the N edge fall back to
// element loads.  A tile is TILE_B / E elements square: 128 bytes of each
// source row and of each destination row, whole 128-byte lines both ways (with
// 64 x 64 one-byte tiles every line was read by two blocks: twice the bytes).
constexpr int TILE_B = 128;
// With 16-byte-aligned LDS rows, rows 16 apart share their banks; the store
// phases read one byte from each of 8 rows 16 apart, so the 16-byte chunks of
// a one-byte tile's row k sit at slot chunk ^ ((k >> 4) & 7) (8 different banks).
__device__ __forceinline__ int tslot(int k, int chunk) { return chunk ^ ((k >> 4) & 7); }
template <int E>
__global__ void __launch_bounds__(256) transpose_tile(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                      int K, int N) {
  constexpr int T = TILE_B / E, V = 16 / E;  // elements per tile side, per 16-byte chunk
  constexpr int ROW = T * E + 16;            // padded LDS row (bytes), 16-byte aligned
  __shared__ __attribute__((aligned(16))) uint8_t tile[T * ROW];
  const int k0 = blockIdx.y * T, n0 = blockIdx.x * T;
  const int t = threadIdx.x;
  for (int idx = t; idx < T * (T / V); idx += 256) {
    const int r = idx / (T / V), c = idx % (T / V);
    const int k = k0 + r, n = n0 + c * V;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (k < K && n < N) {
      const uint8_t* p = src + ((int64_t)k * N + n) * E;
      if (n + V <= N && ((N * E) & 15) == 0) {  // 16-byte aligned rows
        v = *reinterpret_cast<const u32x4*>(p);
      } else {
        uint8_t b[16] = {};
        for (int q = 0; q < min(V, N - n) * E; ++q) b[q] = p[q];
        v = __builtin_bit_cast(u32x4, b);
      }
    }
    *reinterpret_cast<u32x4*>(tile + r * ROW + (E == 1 ? tslot(r, c) : c) * 16) = v;
  }
  __syncthreads();
  for (int idx = t; idx < T * (T / V); idx += 256) {
    const int r = idx / (T / V), c = idx % (T / V);  // r: n, c: chunk of k
    const int n = n0 + r, k = k0 + c * V;
    if (n >= N || k >= K) continue;
    uint8_t b[16];
#pragma unroll
    for (int q = 0; q < V; ++q)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int kr = c * V + q;
        b[q * E + e] = E == 1 ? tile[kr * ROW + tslot(kr, r >> 4) * 16 + (r & 15)] : tile[kr * ROW + r * E + e];
      }
    *reinterpret_cast<u32x4*>(dst + ((int64_t)n * K + k) * E) = __builtin_bit_cast(u32x4, b);
  }
}

// int8 unpack + transpose: packed [K/4, N] -> B^T int8 [N, K] with
// B^T[n, i*K/4 + kb] = ((packed[kb, n] >> 2i) & 3) - 1.  Needs K/4 % 16 == 0.
__global__ void __launch_bounds__(256) unpack_i2_tile(const uint8_t* __restrict__ packed, int8_t* __restrict__ dst,
                                                      int K, int N) {
  constexpr int T = TILE_B, ROW = T + 16;  // 128 packed bytes of a row in, 128 bytes of a quarter row out
  __shared__ __attribute__((aligned(16))) uint8_t tile[T * ROW];
  const int Kb = K / 4;
  const int kb0 = blockIdx.y * T, n0 = blockIdx.x * T;
  const int t = threadIdx.x;
  for (int idx = t; idx < T * (T / 16); idx += 256) {
    const int r = idx / (T / 16), c = idx % (T / 16);
    const int kb = kb0 + r, n = n0 + c * 16;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (kb < Kb && n < N) {
      const uint8_t* p = packed + (int64_t)kb * N + n;
      if (n + 16 <= N && (N & 15) == 0) {  // 16-byte aligned rows
        v = *reinterpret_cast<const u32x4*>(p);
      } else {
        uint8_t b[16] = {};
        for (int q = 0; q < min(16, N - n); ++q) b[q] = p[q];
        v = __builtin_bit_cast(u32x4, b);
      }
    }
    *reinterpret_cast<u32x4*>(tile + r * ROW + tslot(r, c) * 16) = v;
  }
  __syncthreads();
  // output chunk: row n, quarter i, 16 consecutive kb
  for (int idx = t; idx < T * 4 * (T / 16); idx += 256) {
    const int c = idx % (T / 16), i = (idx / (T / 16)) % 4, r = idx / (4 * (T / 16));
    const int n = n0 + r, kb = kb0 + c * 16;
    if (n >= N || kb >= Kb) continue;
    uint32_t w[4];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      uint32_t x = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int kr = c * 16 + q4 * 4 + q;
        x |= (uint32_t)tile[kr * ROW + tslot(kr, r >> 4) * 16 + (r & 15)] << (8 * q);
      }
      // field i of four bytes at once, minus one per byte without carries: (f + 0x7F) ^ 0x80 = f - 1
      w[q4] = (((x >> (2 * i)) & 0x03030303u) + 0x7F7F7F7Fu) ^ 0x80808080u;
    }
    *reinterpret_cast<u32x4*>(dst + (int64_t)n * K + i * Kb + kb) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

// fp32 split for the three-product bf16 GEMM.  A [M, K] -> A' [M, 3K] =
// [hi | hi | lo]; B [K, N] -> B'^T [N, 3K] = [hi^T | lo^T | hi^T].
__device__ __forceinline__ void split_bf16(float x, uint32_t& hi, uint32_t& lo) {
  hi = bf16_bits(x);
  lo = bf16_bits(x - __builtin_bit_cast(float, hi << 16));
}

// four consecutive elements per thread (K % 4 == 0)
__global__ void __launch_bounds__(256) split_rows(const float* __restrict__ A, uint16_t* __restrict__ Ap, int M, int K) {
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_row = K / 4;
  if (v >= (int64_t)M * per_row) return;
  const int64_t m = v / per_row, k = (v - m * per_row) * 4;
  const f32x4 x = *reinterpret_cast<const f32x4*>(A + m * K + k);
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) split_bf16(x[q], hi[q], lo[q]);
  const u32x2 h = {hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
  const u32x2 l = {lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
  uint16_t* row = Ap + m * 3 * K;
  *reinterpret_cast<u32x2*>(row + k) = h;
  *reinterpret_cast<u32x2*>(row + K + k) = h;
  *reinterpret_cast<u32x2*>(row + 2 * K + k) = l;
}

__global__ void __launch_bounds__(256) split_transpose(const float* __restrict__ B, uint16_t* __restrict__ Bp, int K,
                                                       int N) {
  constexpr int T = 64, ROW = T + 4;  // floats
  __shared__ __attribute__((aligned(16))) float tile[T * ROW];
  const int k0 = blockIdx.y * T, n0 = blockIdx.x * T;
  const int t = threadIdx.x;
  for (int idx = t; idx < T * (T / 4); idx += 256) {
    const int r = idx / (T / 4), c = idx % (T / 4);
    const int k = k0 + r, n = n0 + c * 4;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (k < K && n < N) v = *reinterpret_cast<const f32x4*>(B + (int64_t)k * N + n);  // N % 8 == 0
    *reinterpret_cast<f32x4*>(tile + r * ROW + c * 4) = v;
  }
  __syncthreads();
  // output chunk: row n, 8 consecutive k, written to the three segments
  for (int idx = t; idx < T * (T / 8); idx += 256) {
    const int r = idx / (T / 8), c = idx % (T / 8);
    const int n = n0 + r, k = k0 + c * 8;
    if (n >= N || k >= K) continue;
    uint32_t hi[8], lo[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) split_bf16(tile[(c * 8 + q) * ROW + r], hi[q], lo[q]);
    const u32x4 h = {hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16), hi[4] | (hi[5] << 16), hi[6] | (hi[7] << 16)};
    const u32x4 l = {lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16), lo[4] | (lo[5] << 16), lo[6] | (lo[7] << 16)};
    uint16_t* row = Bp + (int64_t)n * 3 * K;
    *reinterpret_cast<u32x4*>(row + k) = h;
    *reinterpret_cast<u32x4*>(row + K + k) = l;
    *reinterpret_cast<u32x4*>(row + 2 * K + k) = h;
  }
}

template <int KIND, int OUT, int BM, int BN, int WM, int WN>
tb_status launch_nt(const uint8_t* A, const uint8_t* BT, void* Y, const float* sa, const float* sw, int64_t M,
                    int64_t N, int64_t Kb, hipStream_t stream, const char* what, int splits = 1) {
  auto kern = &nt_gemm<KIND, OUT, BM, BN, WM, WN>;
  constexpr size_t lds = (size_t)2 * (BM + BN) * BK;
  if (tb_status st = reserve_lds(reinterpret_cast<const void*>(kern), lds, what)) return st;
  const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
  constexpr int threads = (BM / WM) * (BN / WN) * 64;
  hipLaunchKernelGGL(kern, dim3(tiles_m * tiles_n * splits), dim3(threads), lds, stream, A, BT, Y, sa, sw, (int)M,
                     (int)N, (int)Kb, tiles_m, tiles_n, splits);
  return launch_status(what);
}

// Sum of the `splits` int32 partial planes of n elements (n % 4 == 0), in
// plane order, one 16-byte chunk per thread.
__global__ void __launch_bounds__(256) reduce_planes_i32(const i32x4* __restrict__ planes, i32x4* __restrict__ out,
                                                         int64_t n4, int splits) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  i32x4 s = __builtin_nontemporal_load(planes + i);
  for (int p = 1; p < splits; ++p) s += __builtin_nontemporal_load(planes + (int64_t)p * n4 + i);
  out[i] = s;
}

// K splits for the int8 GEMM: 256 x 256 tiles with enough splits to give the
// device about one block per CU, when the 256 x 256 grid alone is too small
// and K is deep enough (at least 8 steps of 128 per split); 1 = no split.
inline int int8_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + 255) / 256) * ((N + 255) / 256);
  if (tiles >= 256) return 1;
  int64_t s = std::min<int64_t>(8, 256 / tiles);
  s = std::min<int64_t>(s, K / BK / 8);
  return s >= 2 ? (int)s : 1;
}

// 256 x 256 tiles when they alone fill the device, else 128 x 128.
inline bool big_tiles(int64_t M, int64_t N) { return ((M + 255) / 256) * ((N + 255) / 256) >= 256; }

}  // namespace ntg
}  // namespace tb

using namespace tb::ntg;

extern "C" tb_status tb_matmul_workspace_size(int dtype, int64_t M, int64_t N, int64_t K, int64_t* bytes) {
  TB_CHECK_ARG(bytes != nullptr, "tb_matmul_workspace_size: null output");
  TB_CHECK_ARG(M > 0 && N > 0 && K > 0, "tb_matmul_workspace_size: sizes must be positive");
  TB_CHECK_ARG(dtype >= 0 && dtype <= 3, "tb_matmul_workspace_size: dtype must be 0 (fp32), 1 (fp16), 2 (fp8) or 3 (int8)");
  switch (dtype) {
    case 0: *bytes = 6 * K * (M + N); break;  // A' and B'^T, bf16, 3K wide
    case 1: *bytes = 2 * K * N; break;        // B^T fp16
    case 2: *bytes = K * N; break;            // B^T e4m3
    default: {                                // unpacked B^T int8, then the split-K partial planes
      *bytes = (K * N + 255) & ~(int64_t)255;
      const int splits = int8_splits(M, N, K);
      if (splits > 1) *bytes += (int64_t)splits * M * N * 4;
      break;
    }
  }
  *bytes = (*bytes + 255) & ~(int64_t)255;
  return TB_OK;
}

extern "C" tb_status tb_matmul_fp8_bt(const uint8_t* a, const uint8_t* bT, uint8_t* out, int64_t M, int64_t N,
                                      int64_t K, hipStream_t stream) {
  TB_CHECK_ARG(a && bT && out, "tb_matmul_fp8_bt: null pointer");
  TB_CHECK_ARG(M > 0 && N > 0 && K > 0, "tb_matmul_fp8_bt: sizes must be positive");
  TB_CHECK_ARG(K % BK == 0 && N % 8 == 0, "tb_matmul_fp8_bt: need K %% 128 == 0 and N %% 8 == 0 (K=%lld N=%lld)",
               (long long)K, (long long)N);
  TB_CHECK_ARG(M * K < (1ll << 31) && N * K < (1ll << 31), "tb_matmul_fp8_bt: operands must be below 2 GiB");
  TB_CHECK_ALIGN(a, 16, "a");
  TB_CHECK_ALIGN(bT, 16, "bT");
  TB_CHECK_ALIGN(out, 4, "out");
  if (big_tiles(M, N))
    return launch_nt<KIND_FP8, OUT_E4M3, 256, 256, 128, 64>(a, bT, out, nullptr, nullptr, M, N, K, stream,
                                                             "tb_matmul_fp8_bt");
  return launch_nt<KIND_FP8, OUT_E4M3, 128, 128, 64, 64>(a, bT, out, nullptr, nullptr, M, N, K, stream,
                                                         "tb_matmul_fp8_bt");
}

extern "C" tb_status tb_matmul(int dtype, const void* a, const void* b, void* out, int64_t M, int64_t N, int64_t K,
                               void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  TB_CHECK_ARG(a && b && out, "tb_matmul: null pointer");
  TB_CHECK_ARG(M > 0 && N > 0 && K > 0, "tb_matmul: sizes must be positive");
  TB_CHECK_ARG(dtype >= 0 && dtype <= 2, "tb_matmul: dtype must be 0 (fp32), 1 (fp16) or 2 (fp8 e4m3)");
  TB_CHECK_ARG(N % 8 == 0, "tb_matmul: N must be a multiple of 8 (got %lld)", (long long)N);
  const int64_t esz = dtype == 0 ? 4 : dtype == 1 ? 2 : 1;
  const int64_t kb = dtype == 0 ? 6 * K : K * esz;  // bytes per operand row in the GEMM
  TB_CHECK_ARG(kb % BK == 0, "tb_matmul: K=%lld is not a multiple of the %lld-element step", (long long)K,
               (long long)(BK / (dtype == 0 ? 2 : esz)));
  TB_CHECK_ARG(M * kb < (1ll << 31) && N * kb < (1ll << 31), "tb_matmul: operands must be below 2 GiB");
  int64_t need = 0;
  tb_matmul_workspace_size(dtype, M, N, K, &need);
  TB_CHECK_ARG(workspace && workspace_bytes >= need, "tb_matmul: needs a %lld-byte workspace (got %lld)",
               (long long)need, (long long)workspace_bytes);
  TB_CHECK_ALIGN(a, 16, "a");
  TB_CHECK_ALIGN(b, 16, "b");
  TB_CHECK_ALIGN(workspace, 256, "workspace");
  TB_CHECK_ALIGN(out, 16, "out");
  const dim3 tgrid((unsigned)((N + 63) / 64), (unsigned)((K + 63) / 64));
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  const bool big = big_tiles(M, N);
  if (dtype == 0) {
    uint16_t* Ap = reinterpret_cast<uint16_t*>(ws);
    uint16_t* Bp = Ap + 3 * M * K;
    hipLaunchKernelGGL(split_rows, dim3((unsigned)((M * (K / 4) + 255) / 256)), dim3(256), 0, stream,
                       reinterpret_cast<const float*>(a), Ap, (int)M, (int)K);
    hipLaunchKernelGGL(split_transpose, tgrid, dim3(256), 0, stream, reinterpret_cast<const float*>(b), Bp, (int)K,
                       (int)N);
    if (big)
      return launch_nt<KIND_BF16, OUT_F32, 256, 256, 128, 64>(reinterpret_cast<const uint8_t*>(Ap),
                                                              reinterpret_cast<const uint8_t*>(Bp), out, nullptr,
                                                              nullptr, M, N, kb, stream, "tb_matmul(fp32)");
    return launch_nt<KIND_BF16, OUT_F32, 128, 128, 64, 64>(reinterpret_cast<const uint8_t*>(Ap),
                                                           reinterpret_cast<const uint8_t*>(Bp), out, nullptr, nullptr,
                                                           M, N, kb, stream, "tb_matmul(fp32)");
  }
  if (dtype == 1) {
    hipLaunchKernelGGL(transpose_tile<2>, tgrid, dim3(256), 0, stream, reinterpret_cast<const uint8_t*>(b), ws,
                       (int)K, (int)N);
    if (big)
      return launch_nt<KIND_F16, OUT_F16, 256, 256, 128, 64>(reinterpret_cast<const uint8_t*>(a), ws, out, nullptr,
                                                             nullptr, M, N, kb, stream, "tb_matmul(fp16)");
    return launch_nt<KIND_F16, OUT_F16, 128, 128, 64, 64>(reinterpret_cast<const uint8_t*>(a), ws, out, nullptr,
                                                          nullptr, M, N, kb, stream, "tb_matmul(fp16)");
  }
  const dim3 tgrid1((unsigned)((N + TILE_B - 1) / TILE_B), (unsigned)((K + TILE_B - 1) / TILE_B));
  hipLaunchKernelGGL(transpose_tile<1>, tgrid1, dim3(256), 0, stream, reinterpret_cast<const uint8_t*>(b), ws, (int)K,
                     (int)N);
  return tb_matmul_fp8_bt(reinterpret_cast<const uint8_t*>(a), ws, reinterpret_cast<uint8_t*>(out), M, N, K, stream);
}

extern "C" tb_status tb_matmul_int8(const int8_t* a, const uint8_t* b, int32_t* out, int64_t M, int64_t N, int64_t K,
                                    void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  TB_CHECK_ARG(a && b && out, "tb_matmul_int8: null pointer");
  TB_CHECK_ARG(M > 0 && N > 0 && K > 0, "tb_matmul_int8: sizes must be positive");
  TB_CHECK_ARG(K % 4 == 0, "tb_matmul_int8: K must be a multiple of 4 (B holds four fields per byte)");
  TB_CHECK_ARG(K % BK == 0 && N % 8 == 0, "tb_matmul_int8: need K %% 128 == 0 and N %% 8 == 0 (K=%lld N=%lld)",
               (long long)K, (long long)N);
  TB_CHECK_ARG(M * K < (1ll << 31) && N * K < (1ll << 31), "tb_matmul_int8: operands must be below 2 GiB");
  int64_t need = 0;
  tb_matmul_workspace_size(3, M, N, K, &need);
  TB_CHECK_ARG(workspace && workspace_bytes >= need, "tb_matmul_int8: needs a %lld-byte workspace (got %lld)",
               (long long)need, (long long)workspace_bytes);
  TB_CHECK_ALIGN(a, 16, "a");
  TB_CHECK_ALIGN(b, 16, "b");
  TB_CHECK_ALIGN(workspace, 256, "workspace");
  TB_CHECK_ALIGN(out, 16, "out");
  int8_t* bt = reinterpret_cast<int8_t*>(workspace);
  hipLaunchKernelGGL(unpack_i2_tile, dim3((unsigned)((N + TILE_B - 1) / TILE_B), (unsigned)((K / 4 + TILE_B - 1) / TILE_B)), dim3(256), 0,
                     stream, b, bt, (int)K, (int)N);
  const int splits = int8_splits(M, N, K);
  if (splits > 1) {
    int32_t* planes = reinterpret_cast<int32_t*>(reinterpret_cast<uint8_t*>(workspace) + ((K * N + 255) & ~(int64_t)255));
    if (tb_status st = launch_nt<KIND_I8, OUT_I32, 256, 256, 128, 64>(
            reinterpret_cast<const uint8_t*>(a), reinterpret_cast<const uint8_t*>(bt), planes, nullptr, nullptr, M, N,
            K, stream, "tb_matmul_int8", splits))
      return st;
    const int64_t n4 = M * N / 4;
    hipLaunchKernelGGL(reduce_planes_i32, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, stream,
                       reinterpret_cast<const i32x4*>(planes), reinterpret_cast<i32x4*>(out), n4, splits);
    return tb::launch_status("tb_matmul_int8(reduce)");
  }
  if (big_tiles(M, N))
    return launch_nt<KIND_I8, OUT_I32, 256, 256, 128, 64>(reinterpret_cast<const uint8_t*>(a),
                                                          reinterpret_cast<const uint8_t*>(bt), out, nullptr, nullptr,
                                                          M, N, K, stream, "tb_matmul_int8");
  return launch_nt<KIND_I8, OUT_I32, 128, 128, 64, 64>(reinterpret_cast<const uint8_t*>(a),
                                                       reinterpret_cast<const uint8_t*>(bt), out, nullptr, nullptr, M,
                                                       N, K, stream, "tb_matmul_int8");
}
