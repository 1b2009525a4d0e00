// Row/column-scaled fp8 GEMM: Y[M, N] = bf16(sa[m] * sw[n] * sum_k Aq[m,k] Wq[k,n]).
//
// Aq is e4m3 [M, K] row-major; the weight operand is passed as WqT [N, K]
// row-major (column n of Wq holds K consecutive bytes: the column-major layout
// torch._scaled_mm takes for its second operand).  fp32 accumulation on the
// CDNA4 fp8 matrix cores (v_mfma_f32_32x32x64_f8f6f4, e4m3 x e4m3), one
// rounding to bf16 (RNE) after both scales.
//
// One 256 x 256 output tile per 512-thread block, eight wavefronts (two per
// SIMD) each owning a 128 x 64 sub-tile (8 fp32 32x32 accumulators), K advanced
// 128 bytes at a time.  Both operands stream HBM -> LDS through the buffer
// unit (buffer_load ... lds, no registers) one step ahead, two LDS stages of
// [256][128 B] per operand.  Rows are split in 16-byte chunks, chunk c of row r
// at slot c ^ ((r ^ (r >> 3)) & 7), so the DMA writes (contiguous) and the
// fragment reads (eight consecutive rows at one chunk) are conflict-free.  A
// fragment of the 32x32x64 MFMA is 32 consecutive bytes of one row (two
// ds_read_b128); A and B use the same k order, which is all a dot product needs.
// The epilogue scales, rounds to bf16, stages the tile in LDS and writes
// 16-byte row chunks.  Tiles are numbered XCD-aware as in the W4A16 kernel.
#include "tb_common.h"

namespace tb {
namespace fp8gemm {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 256, BN = 256, BK = 128, THREADS = 512, GROUP_M = 8;
constexpr int STAGE = BM * BK;  // bytes per operand stage
constexpr int C_STRIDE = BN + 8;  // bf16 elements per staged output row (16-byte pad)
// A and B, two stages each (128 KiB), reused for the staged bf16 output tile.
constexpr size_t LDS_BYTES = 4 * (size_t)STAGE > (size_t)BM * C_STRIDE * 2 ? 4 * (size_t)STAGE
                                                                           : (size_t)BM * C_STRIDE * 2;
constexpr uint32_t RSRC_DW3 = 0x00020000u;
constexpr uint32_t OOB = 0x80000000u;

__device__ __forceinline__ int slot(int row, int chunk) { return row * BK + ((chunk ^ ((row ^ (row >> 3)) & 7)) << 4); }

__device__ __forceinline__ uint16_t bf16_rne(float f) {
  const uint32_t b = __builtin_bit_cast(uint32_t, f);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x40u);
  return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

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

__global__ void __launch_bounds__(THREADS, 1)
    fp8_gemm_kernel(const uint8_t* __restrict__ Aq, const uint8_t* __restrict__ WqT, const float* __restrict__ sa,
                    const float* __restrict__ sw, uint16_t* __restrict__ Y, int M, int N, int K, int tiles_m,
                    int tiles_n) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const Tile tile = tile_of_block(tiles_m, tiles_n);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 2, wn = wave & 3;

  const i32x4 ra = make_rsrc4(Aq, (uint32_t)M * (uint32_t)K);
  const i32x4 rb = make_rsrc4(WqT, (uint32_t)N * (uint32_t)K);
  // DMA: per operand and step, 32 instructions of 1 KiB (8 rows); wave w issues 4.
  uint32_t a_off[4], b_off[4];
  {
    const int lr = lane >> 3;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = (wave * 4 + i) * 8 + lr;
      const int lc = (lane & 7) ^ ((row ^ (row >> 3)) & 7);
      const int m = tile.m0 + row, n = tile.n0 + row;
      a_off[i] = m < M ? (uint32_t)m * (uint32_t)K + (uint32_t)lc * 16u : OOB;
      b_off[i] = n < N ? (uint32_t)n * (uint32_t)K + (uint32_t)lc * 16u : OOB;
    }
  }
  const uint32_t lds0 = (uint32_t)__builtin_amdgcn_readfirstlane(
      (int)(uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  auto issue = [&](int kt) {
    const uint32_t st = lds0 + (uint32_t)((kt & 1) * 2 * STAGE) + (uint32_t)(wave * 4 * 1024);
    const uint32_t soff = (uint32_t)(kt * BK);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(st + i * 1024, a_off[i], ra, soff);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(st + STAGE + i * 1024, b_off[i], rb, soff);
  };

  // Fragment reads: row base + i*32 + (lane & 31); k substep s covers chunks
  // 4s + 2h, 4s + 2h + 1 with h = lane / 32.
  const int a_row = wm * 128 + (lane & 31);
  const int b_row = wn * 64 + (lane & 31);

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  auto frag = [&](const uint8_t* base, int row, int s) -> i32x8 {
    const int c0 = 4 * s + 2 * (lane >> 5);
    const i32x4 lo = *reinterpret_cast<const i32x4*>(base + slot(row, c0));
    const i32x4 hi = *reinterpret_cast<const i32x4*>(base + slot(row, c0 + 1));
    i32x8 r;
    r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
    r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
    return r;
  };

  constexpr int WAIT_VM0 = 0 | (7 << 4) | (15 << 8);
  const int nk = K / BK;
  issue(0);
  __builtin_amdgcn_s_waitcnt(WAIT_VM0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) issue(kt + 1);
    const uint8_t* sa_ = lds + (kt & 1) * 2 * STAGE;
    const uint8_t* sb_ = sa_ + STAGE;
    {
      // Both k64 substeps' fragments are read up front; the scheduling hints
      // then interleave the second substep's 12 LDS reads with the first
      // substep's MFMAs, so the matrix pipe does not wait on LDS latency.
      i32x8 fa0[4], fb0[2], fa1[4], fb1[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) fa0[i] = frag(sa_, a_row + i * 32, 0);
#pragma unroll
      for (int j = 0; j < 2; ++j) fb0[j] = frag(sb_, b_row + j * 32, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) fa1[i] = frag(sa_, a_row + i * 32, 1);
#pragma unroll
      for (int j = 0; j < 2; ++j) fb1[j] = frag(sb_, b_row + j * 32, 1);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa0[i], fb0[j], acc[i][j], 0, 0, 0, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa1[i], fb1[j], acc[i][j], 0, 0, 0, 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);  // substep-0 fragment reads
#pragma unroll
      for (int q = 0; q < 6; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // two substep-1 reads
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 10, 0);
    }
    // Stage kt+1 (issued above, 8 DMA per lane) must land before the barrier
    // that hands it to the next step.
    if (more) __builtin_amdgcn_s_waitcnt(WAIT_VM0);
    __syncthreads();
  }

  // Epilogue: element e of fragment (i, j) is row i*32 + (e/4)*8 + (lane/32)*4 + e%4,
  // column j*32 + lane%32 of the wave tile.
  uint16_t* ct = reinterpret_cast<uint16_t*>(lds);
  const int rbase = wm * 128 + (lane >> 5) * 4;
  const int cbase = wn * 64 + (lane & 31);
  // Scales by buffer loads with out-of-range offsets past M or N (zeros): no
  // branch around a load, so the 66 loads of a lane are in flight together
  // instead of one round trip each.
  const buf_rsrc_t rsa = buf_rsrc(sa, (uint32_t)M * 4u), rsw = buf_rsrc(sw, (uint32_t)N * 4u);
  float swv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = tile.n0 + cbase + j * 32;
    swv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsw, n < N ? (uint32_t)n * 4u : OOB, 0, 0));
  }
  float sav[4][16];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = tile.m0 + rbase + i * 32 + (e >> 2) * 8 + (e & 3);
      sav[i][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsa, m < M ? (uint32_t)m * 4u : OOB, 0, 0));
    }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = rbase + i * 32 + (e >> 2) * 8 + (e & 3);
#pragma unroll
      for (int j = 0; j < 2; ++j) ct[row * C_STRIDE + cbase + j * 32] = bf16_rne(acc[i][j][e] * sav[i][e] * swv[j]);
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
