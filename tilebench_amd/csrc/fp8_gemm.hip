// Row/column-scaled fp8 GEMM: Y[M, N] = bf16(sa[m] * sw[n] * sum_k Aq[m,k] Wq[k,n]).
//
// Aq is e4m3 [M, K] row-major; the weight operand is passed as WqT [N, K]
// row-major (column n of Wq holds K consecutive bytes: the column-major layout
// torch._scaled_mm takes for its second operand).  fp32 accumulation on the
// CDNA4 fp8 matrix cores (v_mfma_f32_32x32x64_f8f6f4, e4m3 x e4m3), one
// rounding to bf16 (RNE) after both scales.
//
// One 256 x 256 output tile per 256-thread block: four wavefronts, one per
// SIMD, each owning a 128 x 128 sub-tile (16 fp32 32x32 accumulators, 256
// accumulator registers).  K advances 128 bytes per step, in two 64-byte
// substeps.  Both operands stream HBM -> LDS through the buffer unit
// (buffer_load ... lds, no registers), two LDS stages of [256][128 B] per
// operand; rows are 16-byte chunks, chunk c of row r at slot
// c ^ ((r ^ (r >> 3)) & 7), so the DMA writes and the fragment reads are
// conflict-free.
//
// The matrix pipe never waits on LDS: while the 16 MFMAs of one substep run,
// the wavefront reads the fragments of the next substep (one ds_read_b128 per
// MFMA).  One barrier per step sits between the two substeps: before it every
// wavefront has finished reading the current stage and has waited for its
// share of the next stage's DMA, so after it the current stage's buffer takes
// the DMA of step k + 2 (issued between the second substep's MFMAs) and the
// next stage's first fragments can be read while the second substep runs.
//
// The MFMA computes the transposed product (W^T fragment first), so a lane
// holds four consecutive output columns of one row per group of four
// accumulator elements; the epilogue scales, rounds to bf16, stages the tile
// in LDS with 8-byte writes and stores 16-byte row chunks.  Tiles are numbered
// XCD-aware as in the W4A16 kernel.
#include "tb_common.h"

#include <type_traits>

namespace tb {
namespace fp8gemm {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

constexpr int BM = 256, BN = 256, BK = 128, THREADS = 256, GROUP_M = 8;
constexpr int STAGE = BM * BK;  // bytes per operand stage
constexpr int C_STRIDE = BN + 8;  // bf16 elements per staged output row (16-byte pad)
// A and B, two stages each (128 KiB), reused for the staged bf16 output tile,
// then the tile's row and column scales (1 KiB each), loaded at the start.
constexpr size_t TILE_BYTES = 4 * (size_t)STAGE > (size_t)BM * C_STRIDE * 2 ? 4 * (size_t)STAGE
                                                                            : (size_t)BM * C_STRIDE * 2;
constexpr size_t SA_OFF = TILE_BYTES, SW_OFF = TILE_BYTES + BM * 4;
constexpr size_t LDS_BYTES = SW_OFF + BN * 4;
static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
constexpr uint32_t RSRC_DW3 = 0x00020000u;
constexpr uint32_t OOB = 0x80000000u;

__device__ __forceinline__ int slot(int row, int chunk) { return row * BK + ((chunk ^ ((row ^ (row >> 3)) & 7)) << 4); }

struct Tile {
  int m0, n0;
};

__device__ __forceinline__ Tile tile_of_block(int tiles_m, int tiles_n) {
  const int nb = tiles_m * tiles_n;
  int bid = blockIdx.x;
  if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  const int per_group = GROUP_M * tiles_n;
  const int group = bid / per_group;
  const int first_m = group * GROUP_M;
  const int rows = min(tiles_m - first_m, GROUP_M);
  const int in_group = bid - group * per_group;
  Tile t;
  t.m0 = (first_m + in_group % rows) * BM;
  t.n0 = (in_group / rows) * BN;
  return t;
}

__device__ __forceinline__ i32x4 make_rsrc4(const void* p, uint32_t bytes) {
  const uint64_t base = (uint64_t)(uintptr_t)p;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)base);
  r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32) & 0xFFFF);
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = (int)RSRC_DW3;
  return r;
}

// One 16-byte-per-lane DMA into LDS at m0 (wave-uniform base, lane l -> +16 l).
// Issued as inline asm so that the compiler does not tie the next barrier to
// its completion; the kernel waits for it explicitly (vmcnt) before the
// barrier that publishes the stage.
__device__ __forceinline__ void dma16(uint32_t lds_addr, uint32_t voff, const i32x4& rsrc, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane((int)lds_addr)), "v"(voff), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane((int)soff))
               : "memory", "m0");
}

// One 4-byte-per-lane DMA into LDS at m0 (lane l -> +4 l).
__device__ __forceinline__ void dma4(uint32_t lds_addr, uint32_t voff, const i32x4& rsrc, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane((int)lds_addr)), "v"(voff), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane((int)soff))
               : "memory", "m0");
}

__global__ void __launch_bounds__(THREADS, 1)
    fp8_gemm_kernel(const uint8_t* __restrict__ Aq, const uint8_t* __restrict__ WqT, const float* __restrict__ sa,
                    const float* __restrict__ sw, uint16_t* __restrict__ Y, int M, int N, int K, int tiles_m,
                    int tiles_n) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const Tile tile = tile_of_block(tiles_m, tiles_n);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const i32x4 ra = make_rsrc4(Aq, (uint32_t)M * (uint32_t)K);
  const i32x4 rb = make_rsrc4(WqT, (uint32_t)N * (uint32_t)K);
  // the DMAs issued past the last step read through empty resources: zeros,
  // no memory traffic, nothing for the epilogue to wait on
  const i32x4 ra0 = make_rsrc4(Aq, 0u), rb0 = make_rsrc4(WqT, 0u);
  // DMA: per operand and stage, 32 instructions of 1 KiB (8 rows); wave w issues 8 of each.
  uint32_t a_off[8], b_off[8];
  {
    const int lr = lane >> 3;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = (wave * 8 + i) * 8 + lr;
      const int lc = (lane & 7) ^ ((row ^ (row >> 3)) & 7);
      const int m = tile.m0 + row, n = tile.n0 + row;
      a_off[i] = m < M ? (uint32_t)m * (uint32_t)K + (uint32_t)lc * 16u : OOB;
      b_off[i] = n < N ? (uint32_t)n * (uint32_t)K + (uint32_t)lc * 16u : OOB;
    }
  }
  const uint32_t lds0 = (uint32_t)__builtin_amdgcn_readfirstlane(
      (int)(uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  // LDS layout [A stage 0 | A stage 1 | B stage 0 | B stage 1], 32 KiB each.
  // DMA instruction q (0..15) of step kt: A rows for q < 8, B rows for q >= 8.
  const int nk = K / BK;
  auto dma = [&](int kt, int q) {
    const uint32_t st = lds0 + (uint32_t)((kt & 1) * STAGE) + (uint32_t)(wave * 8 * 1024);
    const uint32_t soff = (uint32_t)(kt * BK);
    const bool live = kt < nk;
    if (q < 8)
      dma16(st + q * 1024, a_off[q], live ? ra : ra0, soff);
    else
      dma16(st + 2 * STAGE + (q - 8) * 1024, b_off[q - 8], live ? rb : rb0, soff);
  };

  // Fragment f (0..3 A rows, 4..7 B rows) of substep s: row base + (f & 3) * 32
  // + lane % 32, chunks 4s + 2h and 4s + 2h + 1 with h = lane / 32 (32 bytes).
  // Rows 32 apart differ in bit 2 of (row >> 3) only, so the swizzle depends on
  // f & 1: per operand, substep and half, two base addresses (f even / odd)
  // cover all four fragments with immediate offsets (8 KiB apart), and the
  // stage (32 KiB) is an immediate too.
  const int a_row = wm * 128 + (lane & 31);
  const int b_row = wn * 128 + (lane & 31);
  uint32_t abase[2][2][2], bbase[2][2][2];  // [s][half][f & 1]
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int par = 0; par < 2; ++par) {
        const int c = 4 * s2 + 2 * (lane >> 5) + hf;
        abase[s2][hf][par] = (uint32_t)slot(a_row + par * 32, c);
        bbase[s2][hf][par] = (uint32_t)(2 * STAGE + slot(b_row + par * 32, c));
      }
  auto frag = [&](auto stage, int f, int s2) -> i32x8 {
    constexpr int ST = decltype(stage)::value * STAGE;
    const uint32_t* bs = f < 4 ? &abase[s2][0][0] : &bbase[s2][0][0];
    const int par = f & 1, off = ST + ((f & 3) >> 1) * 8192;
    const i32x4 lo = *reinterpret_cast<const i32x4*>(lds + bs[0 * 2 + par] + off);
    const i32x4 hi = *reinterpret_cast<const i32x4*>(lds + bs[1 * 2 + par] + off);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  // Fragment registers of one substep: 4 A and 4 B fragments of 8 dwords.
  i32x8 cur[8], nxt[8];
  // 16 MFMAs (4 A x 4 B fragments); after MFMA q, body(q) issues interleaved work.
  auto mfma_all = [&](i32x8 (&fr)[8], auto body) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // transposed product: W^T fragment first, so a lane holds 4 consecutive columns
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fr[4 + j], fr[i], acc[i][j], 0, 0, 0, 0, 0, 0);
        body(i * 4 + j);
      }
  };

  constexpr int WAIT_VM0 = 0 | (7 << 4) | (15 << 8);
  constexpr int WAIT_VM16_LGKM0 = 0 | (7 << 4) | (0 << 8) | (1 << 14);  // vmcnt(16), lgkmcnt(0)
  // Prologue: the tile's scales (wave w: rows and columns 64w .. 64w + 63;
  // zeros past M or N), then stages 0 and 1 in flight, wait for stage 0, read
  // its substep-0 fragments.
  {
    const i32x4 rsa = make_rsrc4(sa, (uint32_t)M * 4u), rsw = make_rsrc4(sw, (uint32_t)N * 4u);
    const int m = tile.m0 + wave * 64 + lane, n = tile.n0 + wave * 64 + lane;
    dma4(lds0 + (uint32_t)(SA_OFF + wave * 256), m < M ? (uint32_t)m * 4u : OOB, rsa, 0u);
    dma4(lds0 + (uint32_t)(SW_OFF + wave * 256), n < N ? (uint32_t)n * 4u : OOB, rsw, 0u);
  }
#pragma unroll
  for (int q = 0; q < 16; ++q) dma(0, q);
  if (nk > 1) {
#pragma unroll
    for (int q = 0; q < 16; ++q) dma(1, q);
    __builtin_amdgcn_s_waitcnt(WAIT_VM16_LGKM0);
  } else {
    __builtin_amdgcn_s_waitcnt(WAIT_VM0);
  }
  __syncthreads();
#pragma unroll
  for (int f = 0; f < 8; ++f) cur[f] = frag(std::integral_constant<int, 0>{}, f, 0);

  // Step kt on stage SB = kt & 1 (a compile-time constant: the loop runs two
  // steps per iteration).
  auto step = [&](int kt, auto sbc) {
    constexpr int SB = decltype(sbc)::value;
    const std::integral_constant<int, SB> cur_st{};
    const std::integral_constant<int, SB ^ 1> nxt_st{};
    // substep 0: MFMAs on `cur`; one fragment of substep 1 of this stage read
    // into `nxt` after every second MFMA.  The scheduling barriers keep this
    // order: MFMAs are asynchronous, so the reads go out while they run.
    mfma_all(cur, [&](int q) {
      if ((q & 1) == 0) nxt[q >> 1] = frag(cur_st, q >> 1, 1);
      __builtin_amdgcn_sched_barrier(0);
    });
    // this stage is fully read; the next one must have landed (each wave waits
    // for its own DMA, the barrier publishes all of them)
    __builtin_amdgcn_s_waitcnt(WAIT_VM0);
    __syncthreads();
    // substep 1: MFMAs on `nxt`; the next stage's substep-0 fragments read into
    // `cur`; the DMA of step kt + 2 refills this stage's buffer.  Past the last
    // steps both still go out: a stale stage is read into registers nobody
    // uses, and the DMA past K fetches in-bounds bytes (or zeros past the
    // buffer) into a stage nobody reads.
    mfma_all(nxt, [&](int q) {
      if ((q & 1) == 0) cur[q >> 1] = frag(nxt_st, q >> 1, 0);
      dma(kt + 2, q);
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  int kt = 0;
  for (; kt + 1 < nk; kt += 2) {
    step(kt, std::integral_constant<int, 0>{});
    step(kt + 1, std::integral_constant<int, 1>{});
  }
  if (kt < nk) step(kt, std::integral_constant<int, 0>{});
  __builtin_amdgcn_s_waitcnt(WAIT_VM0);  // the DMAs issued past the end, before LDS is reused

  // Epilogue: with the transposed product, element e of fragment (i, j) is
  // row i*32 + lane%32, column j*32 + (e/4)*8 + (lane/32)*4 + e%4 of the wave tile.
  __syncthreads();  // every wave is done with the stages before they hold the output tile
  uint16_t* ct = reinterpret_cast<uint16_t*>(lds);
  // scales from LDS (landed before the first K step's barrier)
  const float* lsa = reinterpret_cast<const float*>(lds + SA_OFF);
  const float* lsw = reinterpret_cast<const float*>(lds + SW_OFF);
  float sav[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sav[i] = lsa[wm * 128 + i * 32 + (lane & 31)];
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  typedef float f32x2v __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
  f32x4v swv[4][4];  // [j][g]: columns j*32 + g*8 + (lane/32)*4 + 0..3
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      swv[j][g] = *reinterpret_cast<const f32x4v*>(lsw + wn * 128 + j * 32 + g * 8 + (lane >> 5) * 4);
  // (acc * sa) * sw in fp32, then one RNE rounding to bf16 by the hardware
  // converter (v_cvt_pk_bf16_f32)
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int row = wm * 128 + i * 32 + (lane & 31);
        const int col = wn * 128 + j * 32 + g * 8 + (lane >> 5) * 4;
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = acc[i][j][4 * g + e] * sav[i] * swv[j][g][e];
        u32x2v v;
        v[0] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v{f[0], f[1]}), bf16x2v));
        v[1] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v{f[2], f[3]}), bf16x2v));
        *reinterpret_cast<u32x2v*>(ct + row * C_STRIDE + col) = v;
      }
  __syncthreads();
  const int rows = min(BM, M - tile.m0);
  const int cols = min(BN, N - tile.n0);
  for (int idx = t; idx < BM * (BN / 8); idx += THREADS) {
    const int row = idx >> 5, ch = idx & 31;
    if (row < rows && ch * 8 < cols) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(ct + row * C_STRIDE + ch * 8);
      *reinterpret_cast<u32x4*>(Y + (int64_t)(tile.m0 + row) * N + tile.n0 + ch * 8) = v;
    }
  }
}

}  // namespace fp8gemm
}  // namespace tb

extern "C" tb_status tb_fp8_scaled_gemm(const uint8_t* Aq, const uint8_t* WqT, const float* sa, const float* sw,
                                        uint16_t* Y, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  using namespace tb::fp8gemm;
  TB_CHECK_ARG(Aq && WqT && sa && sw && Y, "tb_fp8_scaled_gemm: null pointer");
  TB_CHECK_ARG(M > 0 && N > 0 && K > 0, "tb_fp8_scaled_gemm: sizes must be positive");
  TB_CHECK_ARG(K % BK == 0, "tb_fp8_scaled_gemm: K must be a multiple of %d (got %lld)", BK, (long long)K);
  TB_CHECK_ARG(N % 8 == 0, "tb_fp8_scaled_gemm: N must be a multiple of 8 (got %lld)", (long long)N);
  TB_CHECK_ARG(M * K < (1ll << 31) && N * K < (1ll << 31),
               "tb_fp8_scaled_gemm: each operand must be smaller than 2 GiB (M=%lld N=%lld K=%lld)", (long long)M,
               (long long)N, (long long)K);
  TB_CHECK_ALIGN(Aq, 16, "Aq");
  TB_CHECK_ALIGN(WqT, 16, "WqT");
  TB_CHECK_ALIGN(Y, 16, "Y");
  if (tb_status st = tb::reserve_lds(reinterpret_cast<const void*>(&fp8_gemm_kernel), LDS_BYTES, "tb_fp8_scaled_gemm"))
    return st;
  const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
  hipLaunchKernelGGL(fp8_gemm_kernel, dim3(tiles_m * tiles_n), dim3(THREADS), LDS_BYTES, stream, Aq, WqT, sa, sw, Y,
                     (int)M, (int)N, (int)K, tiles_m, tiles_n);
  return tb::launch_status("tb_fp8_scaled_gemm");
}
