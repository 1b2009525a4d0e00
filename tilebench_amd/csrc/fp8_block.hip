// Block-scaled fp8-e4m3 (the 128 x 128 weight blocks of DeepSeek-V3-style fp8
// checkpoints, with activations quantised per token and per 128 input
// channels):
//
//   tb_fp8_act_quant_blocks   sa[kb, m] = fp32(max_{k in block kb} |A[m,k]|) / 448
//                             Aq[m, k]  = e4m3(RN32(fp32(A[m,k]) / sa[k/128, m]))
//                             the per-token quantiser's arithmetic (fp8_codec.h) on
//                             each 128-element block of a row; sa is stored
//                             block-major ([K/128, M], M contiguous).
//   tb_fp8_block_gemm         Y[m, n] = bf16( sum_kb (sa[kb, m] * sw[n/128, kb]) * P_kb[m, n] ),
//                             P_kb = sum_{k in block kb} Aq[m,k] * WqT[n,k] in fp32 on the
//                             fp8 matrix cores; the scaled block sums are added in fp32
//                             in block order.  sw is the checkpoint's weight_scale_inv
//                             layout, [ceil(N/128), K/128] row-major.
//
// GEMM structure.  One 256 x 128 output tile per 256-thread block: four
// wavefronts, one per SIMD, each owning 128 x 64 (4 x 2 fragments of 32 x 32).
// A K step is 128 bytes = one scale block.  Operands stream HBM -> LDS by DMA
// (buffer_load ... lds) one step ahead into two stages, with the row swizzle
// of the other fp8 kernels (chunk c of row r at slot c ^ ((r ^ (r >> 3)) & 7)).
// Per step and fragment pair (i, j) two MFMAs (k 0..63 and 64..127) start from
// zero and give P_kb; one fp32 FMA per element adds s_i * P_kb to the
// accumulator, s_i = sa * sw of the lane's row in fragment row i (the tile's
// 128 columns are one weight block, so sw is one value per step).  The step's
// 256 activation scales go HBM -> LDS with the operands, permuted so that a
// lane reads its four rows' scales with one 16-byte LDS read; the tile's
// column of weight scales (K/128 values) is loaded once at the start.
#include "tb_common.h"
#include "fp8_codec.h"

namespace tb {
namespace fp8blk {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

constexpr int BM = 256, BN = 128, BK = 128, WM = 128, WN = 64, WAVES = 4, THREADS = 256;
constexpr int FI = WM / 32, FJ = WN / 32;
constexpr int A_STAGE = BM * BK, B_STAGE = BN * BK, STAGE = A_STAGE + B_STAGE;
constexpr int A_DMA = BM / 8 / WAVES, B_DMA = BN / 8 / WAVES;  // 1 KiB DMA instructions per wave and step
constexpr int MAX_KB = 512;                                     // K <= 65536
constexpr size_t SA_OFF = 2 * (size_t)STAGE, SW_OFF = SA_OFF + 2 * BM * 4;
constexpr size_t LDS_BYTES = SW_OFF + MAX_KB * 4;
static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
static_assert(A_DMA * WAVES * 8 == BM && B_DMA * WAVES * 8 == BN, "tile rows must split evenly over the DMA");
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

// DMAs into LDS at m0 (wave-uniform base; lane l lands at +16 l or +4 l), as
// inline asm so that the compiler does not tie barriers to their completion;
// the kernel waits for them (vmcnt) before the barrier that publishes them.
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

// Tiles in groups of 8 tile rows, column-major inside a group; with the tile
// count a multiple of 8, the blocks one XCD receives (every 8th block id) are
// one contiguous run of tiles, so an XCD's L2 serves neighbouring tiles.
__device__ __forceinline__ void tile_of_block(int tiles_m, int tiles_n, int& m0, int& n0) {
  constexpr int GROUP_M = 8;
  const int nb = tiles_m * tiles_n;
  int bid = (int)blockIdx.x;
  if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  const int per_group = GROUP_M * tiles_n;
  const int group = bid / per_group;
  const int first_m = group * GROUP_M;
  const int rows = min(tiles_m - first_m, GROUP_M);
  const int in_group = bid - group * per_group;
  m0 = (first_m + in_group % rows) * BM;
  n0 = (in_group / rows) * BN;
}

__global__ void __launch_bounds__(THREADS, 1)
    fp8_block_gemm(const uint8_t* __restrict__ Aq, const uint8_t* __restrict__ WqT, const float* __restrict__ sa,
                   const float* __restrict__ sw, uint16_t* __restrict__ Y, int M, int N, int K, int tiles_m,
                   int tiles_n) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  int m0, n0;
  tile_of_block(tiles_m, tiles_n, m0, n0);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int nkb = K / BK;

  const i32x4 ra = make_rsrc4(Aq, (uint32_t)M * (uint32_t)K);
  const i32x4 rb = make_rsrc4(WqT, (uint32_t)N * (uint32_t)K);
  const i32x4 rsa = make_rsrc4(sa, (uint32_t)nkb * (uint32_t)M * 4u);
  const int nb = n0 / BN;  // this tile's weight-scale block row (BN = 128)
  const i32x4 rsw = make_rsrc4(sw, (uint32_t)((N + 127) / 128) * (uint32_t)nkb * 4u);
  uint32_t a_off[A_DMA], b_off[B_DMA];
  {
    const int lr = lane >> 3;
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) {
      const int row = (wave * A_DMA + i) * 8 + lr;
      const int lc = (lane & 7) ^ ((row ^ (row >> 3)) & 7);
      a_off[i] = m0 + row < M ? (uint32_t)(m0 + row) * (uint32_t)K + (uint32_t)lc * 16u : OOB;
    }
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) {
      const int row = (wave * B_DMA + i) * 8 + lr;
      const int lc = (lane & 7) ^ ((row ^ (row >> 3)) & 7);
      b_off[i] = n0 + row < N ? (uint32_t)(n0 + row) * (uint32_t)K + (uint32_t)lc * 16u : OOB;
    }
  }
  // Activation scales of a step: LDS float p = 64 wave + lane holds the scale
  // of tile row 128 (p / 128) + 32 (p % 4) + (p % 128) / 4, so that the lane
  // (wm, c = lane % 32) finds its rows wm*128 + 32 i + c (i = 0..3) at
  // 128 wm + 4 c + i: one 16-byte read.
  uint32_t sa_off;
  {
    const int p = wave * 64 + lane;
    const int row = (p >> 7) * 128 + 32 * (p & 3) + ((p & 127) >> 2);
    sa_off = m0 + row < M ? (uint32_t)(m0 + row) * 4u : OOB;
  }
  const uint32_t lds0 = (uint32_t)__builtin_amdgcn_readfirstlane(
      (int)(uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  auto issue = [&](int kt) {
    const uint32_t st = lds0 + (uint32_t)((kt & 1) * STAGE);
    const uint32_t soff = (uint32_t)(kt * BK);
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) dma16(st + (uint32_t)((wave * A_DMA + i) * 1024), a_off[i], ra, soff);
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) dma16(st + A_STAGE + (uint32_t)((wave * B_DMA + i) * 1024), b_off[i], rb, soff);
    dma4(lds0 + (uint32_t)(SA_OFF + (kt & 1) * BM * 4 + wave * 256), sa_off, rsa, (uint32_t)kt * (uint32_t)M * 4u);
  };
  // The tile's weight scales sw[nb, 0 .. nkb-1]: wave w loads entries 64 q + lane for q = w, w + 4, ...
  for (int q = wave; q * 64 < nkb; q += WAVES) {
    const int kb = q * 64 + lane;
    dma4(lds0 + (uint32_t)(SW_OFF + q * 256), kb < nkb ? (uint32_t)kb * 4u : OOB, rsw,
         (uint32_t)nb * (uint32_t)nkb * 4u);
  }

  const int a_row = wm * WM + (lane & 31);
  const int b_row = wn * WN + (lane & 31);
  // fragment of substep s (32 bytes: chunks 4s + 2h and 4s + 2h + 1, h = lane / 32)
  auto frag = [&](const uint8_t* base, int row, int s) -> i32x8 {
    const int c0 = 4 * s + 2 * (lane >> 5);
    const i32x4 lo = *reinterpret_cast<const i32x4*>(base + slot(row, c0));
    const i32x4 hi = *reinterpret_cast<const i32x4*>(base + slot(row, c0 + 1));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };

  f32x16 acc[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j) acc[i][j] = f32x16{};

  constexpr int WAIT_VM0 = 0 | (7 << 4) | (15 << 8);
  const float* lsw = reinterpret_cast<const float*>(lds + SW_OFF);
  issue(0);
  __builtin_amdgcn_s_waitcnt(WAIT_VM0);
  __syncthreads();
  for (int kt = 0; kt < nkb; ++kt) {
    const bool more = kt + 1 < nkb;
    if (more) issue(kt + 1);
    const uint8_t* sa_ = lds + (kt & 1) * STAGE;
    const uint8_t* sb_ = sa_ + A_STAGE;
    i32x8 fa0[FI], fa1[FI], fb0[FJ], fb1[FJ];
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
      fb0[j] = frag(sb_, b_row + j * 32, 0);
      fb1[j] = frag(sb_, b_row + j * 32, 1);
    }
#pragma unroll
    for (int i = 0; i < FI; ++i) {
      fa0[i] = frag(sa_, a_row + i * 32, 0);
      fa1[i] = frag(sa_, a_row + i * 32, 1);
    }
    const f32x4 sav = *reinterpret_cast<const f32x4*>(lds + SA_OFF + (kt & 1) * BM * 4 + (wm * 128 + 4 * (lane & 31)) * 4);
    const float swv = lsw[kt];
    float s[FI];
#pragma unroll
    for (int i = 0; i < FI; ++i) s[i] = sav[i] * swv;
#pragma unroll
    for (int i = 0; i < FI; ++i)
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
        // transposed product (W^T fragment first): a lane holds 4 consecutive columns
        f32x16 p = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb0[j], fa0[i], f32x16{}, 0, 0, 0, 0, 0, 0);
        p = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb1[j], fa1[i], p, 0, 0, 0, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = __builtin_fmaf(p[e], s[i], acc[i][j][e]);
      }
    // stage kt + 1 must land before the barrier that hands it to the next step
    if (more) __builtin_amdgcn_s_waitcnt(WAIT_VM0);
    __syncthreads();
  }

  // Epilogue straight from registers: elements 4g .. 4g+3 of fragment (i, j)
  // are row i*32 + lane%32, columns j*32 + g*8 + (lane/32)*4 + 0..3 of the wave
  // tile (N % 8 == 0: four columns are all in or all out).  One RNE rounding
  // to bf16 by the hardware converter.
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
        u32x2 v;
        v[0] = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                                                (f32x2v{acc[i][j][4 * g], acc[i][j][4 * g + 1]}), bf16x2v));
        v[1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                                                (f32x2v{acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]}), bf16x2v));
        *reinterpret_cast<u32x2*>(Y + (int64_t)m * N + n) = v;
      }
  }
}

// ------------------------------------------------------------------ activation quantiser

// One 16-lane group per 128-element block of a row (a lane holds 8 halfs),
// four blocks per wavefront, 16 per 256-thread block; the blocks of a row are
// consecutive, so a wavefront reads 1 KiB of one row (or of two rows at a
// row boundary) per load.
__global__ void __launch_bounds__(256) fp8_quant_blocks(const u32x4* __restrict__ A, u32x2* __restrict__ Aq,
                                                        float* __restrict__ sa_out, int64_t M, int64_t nkb) {
  const int64_t blk = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);  // global block id = m * nkb + kb
  const int sub = threadIdx.x & 15;
  const int64_t total = M * nkb;
  const bool live = blk < total;
  const buf_rsrc_t rs = buf_rsrc(A, (uint32_t)min<int64_t>(total * 256, 0x7FFFFFFFll));
  const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rs, live ? (uint32_t)((blk * 16 + sub) * 16) : BUF_OOB, 0,
                                                        2 /* nt */);
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t a = x[j] & 0x7FFF7FFFu;
    m = max(m, max(a & 0xFFFFu, a >> 16));
  }
  // maximum over the 16 lanes of the group (xor partners stay inside it)
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off, 64));
  const float amax = (float)__builtin_bit_cast(_Float16, (uint16_t)m);
  const float s = amax / 448.0f;
  const float y = 1.0f / s;
  if (!live) return;
  const int64_t row = blk / nkb, kb = blk - row * nkb;
  if (sub == 0) sa_out[kb * M + row] = s;
  Aq[blk * 16 + sub] = quantize_chunk(x, s, y, m);
}

}  // namespace fp8blk
}  // namespace tb

extern "C" tb_status tb_fp8_act_quant_blocks(const uint16_t* A, uint8_t* Aq, float* sa, int64_t M, int64_t K,
                                             hipStream_t stream) {
  TB_CHECK_ARG(A && Aq && sa, "tb_fp8_act_quant_blocks: null pointer");
  TB_CHECK_ARG(M > 0 && K > 0 && K % 128 == 0,
               "tb_fp8_act_quant_blocks: need M > 0 and K a positive multiple of 128 (M=%lld K=%lld)", (long long)M,
               (long long)K);
  TB_CHECK_ARG(M * K * 2 < (1ll << 31), "tb_fp8_act_quant_blocks: A must be smaller than 2 GiB");
  TB_CHECK_ALIGN(A, 16, "A");
  TB_CHECK_ALIGN(Aq, 8, "Aq");
  const int64_t blocks = M * (K / 128);
  hipLaunchKernelGGL(tb::fp8blk::fp8_quant_blocks, dim3((unsigned)((blocks + 15) / 16)), dim3(256), 0, stream,
                     reinterpret_cast<const tb::u32x4*>(A), reinterpret_cast<tb::u32x2*>(Aq), sa, M, K / 128);
  return tb::launch_status("tb_fp8_act_quant_blocks");
}

extern "C" tb_status tb_fp8_block_gemm(const uint8_t* Aq, const uint8_t* WqT, const float* sa, const float* sw,
                                       uint16_t* Y, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  using namespace tb::fp8blk;
  TB_CHECK_ARG(Aq && WqT && sa && sw && Y, "tb_fp8_block_gemm: null pointer");
  TB_CHECK_ARG(M > 0 && N > 0 && K > 0, "tb_fp8_block_gemm: sizes must be positive");
  TB_CHECK_ARG(K % BK == 0 && K / BK <= MAX_KB,
               "tb_fp8_block_gemm: K must be a multiple of %d and at most %d (got %lld)", BK, BK * MAX_KB,
               (long long)K);
  TB_CHECK_ARG(N % 8 == 0, "tb_fp8_block_gemm: N must be a multiple of 8 (got %lld)", (long long)N);
  TB_CHECK_ARG(M * K < (1ll << 31) && N * K < (1ll << 31) && (K / BK) * M * 4 < (1ll << 31),
               "tb_fp8_block_gemm: each operand must be smaller than 2 GiB (M=%lld N=%lld K=%lld)", (long long)M,
               (long long)N, (long long)K);
  TB_CHECK_ALIGN(Aq, 16, "Aq");
  TB_CHECK_ALIGN(WqT, 16, "WqT");
  TB_CHECK_ALIGN(sa, 4, "sa");
  TB_CHECK_ALIGN(sw, 4, "sw");
  TB_CHECK_ALIGN(Y, 8, "Y");
  if (tb_status st = tb::reserve_lds(reinterpret_cast<const void*>(&fp8_block_gemm), LDS_BYTES, "tb_fp8_block_gemm"))
    return st;
  const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
  hipLaunchKernelGGL(fp8_block_gemm, dim3(tiles_m * tiles_n), dim3(THREADS), LDS_BYTES, stream, Aq, WqT, sa, sw, Y,
                     (int)M, (int)N, (int)K, tiles_m, tiles_n);
  return tb::launch_status("tb_fp8_block_gemm");
}
