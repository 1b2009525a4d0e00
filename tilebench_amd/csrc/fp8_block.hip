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
// GEMM structure.  One 256 x 256 output tile per 512-thread block: eight
// wavefronts, two per SIMD, each owning 128 x 64 (4 x 2 fragments of 32 x 32;
// 128 fp32 accumulator registers, all in VGPRs because the VALU adds into
// them).  A K step is 128 bytes = one scale block.  Operands stream HBM -> LDS
// by DMA (buffer_load ... lds) one step ahead into two stages, with the row
// swizzle of the other fp8 kernels (chunk c of row r at slot
// c ^ ((r ^ (r >> 3)) & 7)); DMAs past the last step go through empty
// resources, so the loop has no branch.  Per step and fragment pair (i, j)
// two MFMAs (k 0..63 and 64..127) start from zero and give P_kb (in VGPRs:
// the file is compiled with the VGPR form of the MFMAs); one fp32 FMA per
// element adds s_i * P_kb to the accumulator, s_i = sa * sw of the lane's row
// in fragment row i (a wavefront's 64 columns lie in one weight block, so sw
// is one value per step).  The FMAs of pair q - 1 are issued between the MFMAs
// of pair q (the matrix pipe and the VALU work side by side; at most two block
// sums are live).  The step's 256 activation scales go HBM -> LDS with the
// operands, permuted so that a lane reads its four rows' scales with one
// 16-byte LDS read; the tile's two columns of weight scales (K/128 values
// each) are loaded once at the start.
#include "tb_common.h"
#include "fp8_codec.h"

namespace tb {
namespace fp8blk {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

constexpr int BM = 256, BK = 128, WM = 128, WN = 64;
constexpr int FI = WM / 32, FJ = WN / 32;
constexpr int MAX_KB = 512;  // K <= 65536

// Tile configuration: BN columns (128 or 256), WAVES wavefronts of WM x WN,
// NSTAGE operand stages in LDS (the DMA runs NSTAGE - 1 steps ahead).
template <int BN, int WAVES, int NSTAGE>
struct Cfg {
  static constexpr int THREADS = WAVES * 64;
  static constexpr int A_STAGE = BM * BK, B_STAGE = BN * BK, STAGE = A_STAGE + B_STAGE;
  static constexpr int A_DMA = BM / 8 / WAVES, B_DMA = BN / 8 / WAVES;  // 1 KiB DMAs per wave and step
  static constexpr int SW_BLOCKS = BN / 128;                            // weight-scale blocks per tile
  static constexpr size_t SA_OFF = NSTAGE * (size_t)STAGE;              // NSTAGE x 256 activation scales
  static constexpr size_t DUMP_OFF = SA_OFF + NSTAGE * BM * 4;          // target of the idle waves' scale DMA
  static constexpr size_t SW_OFF = DUMP_OFF + 256;                      // SW_BLOCKS x MAX_KB weight scales
  static constexpr size_t LDS_BYTES = SW_OFF + (size_t)SW_BLOCKS * MAX_KB * 4;
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
  static_assert(A_DMA * WAVES * 8 == BM && B_DMA * WAVES * 8 == BN, "tile rows must split evenly over the DMA");
  static_assert((BM / WM) * (BN / WN) == WAVES, "wave grid");
};
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
template <int BN>
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

template <int BN, int WAVES, int NSTAGE>
__global__ void __launch_bounds__(WAVES * 64, 1)
    fp8_block_gemm(const uint8_t* __restrict__ Aq, const uint8_t* __restrict__ WqT, const float* __restrict__ sa,
                   const float* __restrict__ sw, uint16_t* __restrict__ Y, int M, int N, int K, int tiles_m,
                   int tiles_n) {
  typedef Cfg<BN, WAVES, NSTAGE> C;
  constexpr int A_STAGE = C::A_STAGE, STAGE = C::STAGE, A_DMA = C::A_DMA, B_DMA = C::B_DMA;
  constexpr size_t SA_OFF = C::SA_OFF, SW_OFF = C::SW_OFF;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  int m0, n0;
  tile_of_block<BN>(tiles_m, tiles_n, m0, n0);
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: LDS and DMA bases stay scalar
  const int wm = wave / (BN / WN), wn = wave % (BN / WN);
  const int nkb = K / BK;

  const i32x4 ra = make_rsrc4(Aq, (uint32_t)M * (uint32_t)K);
  const i32x4 rb = make_rsrc4(WqT, (uint32_t)N * (uint32_t)K);
  const i32x4 rsa = make_rsrc4(sa, (uint32_t)nkb * (uint32_t)M * 4u);
  const int nbN = (N + 127) / 128;  // weight-scale block rows
  const i32x4 rsw = make_rsrc4(sw, (uint32_t)nbN * (uint32_t)nkb * 4u);
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
  // Waves 4 and up have no scales to load; they issue the same DMA through an
  // empty resource into a dump area, so every wave counts the same DMAs.
  uint32_t sa_off;
  {
    const int p = wave * 64 + lane;
    const int row = (p >> 7) * 128 + 32 * (p & 3) + ((p & 127) >> 2);
    sa_off = wave < 4 && m0 + row < M ? (uint32_t)(m0 + row) * 4u : OOB;
  }
  const uint32_t lds0 = (uint32_t)__builtin_amdgcn_readfirstlane(
      (int)(uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  // DMAs of a step past the last one go through resources of size 0: they
  // read nothing and fill a stage no step reads, so every step issues the same
  // DMAs and waits the same way (no branch in the loop).
  const i32x4 ra0 = make_rsrc4(Aq, 0u), rb0 = make_rsrc4(WqT, 0u), rsa0 = make_rsrc4(sa, 0u);
  auto issue = [&](int kt) {
    const int sidx = kt % NSTAGE;
    const bool live = kt < nkb;
    const uint32_t st = lds0 + (uint32_t)(sidx * STAGE);
    const uint32_t soff = live ? (uint32_t)(kt * BK) : 0u;
#pragma unroll
    for (int i = 0; i < A_DMA; ++i)
      dma16(st + (uint32_t)((wave * A_DMA + i) * 1024), a_off[i], live ? ra : ra0, soff);
#pragma unroll
    for (int i = 0; i < B_DMA; ++i)
      dma16(st + A_STAGE + (uint32_t)((wave * B_DMA + i) * 1024), b_off[i], live ? rb : rb0, soff);
    const bool scales = wave < 4;
    dma4(lds0 + (uint32_t)(scales ? SA_OFF + sidx * BM * 4 + wave * 256 : C::DUMP_OFF), sa_off,
         live && scales ? rsa : rsa0, live ? (uint32_t)kt * (uint32_t)M * 4u : 0u);
  };
  constexpr int DMA_PER_STEP = A_DMA + B_DMA + 1;  // per wavefront
  // The tile's weight scales sw[n0 / 128 + b, 0 .. nkb-1] (b < BN / 128) at
  // LDS float b * MAX_KB + kb: instruction q = b * nq + c loads kb = 64 c + lane.
  {
    const int nq = (nkb + 63) / 64;
    for (int q = wave; q < C::SW_BLOCKS * nq; q += WAVES) {
      const int b = q / nq, kb = (q % nq) * 64 + lane, nb = n0 / 128 + b;
      dma4(lds0 + (uint32_t)(SW_OFF + b * MAX_KB * 4 + (q % nq) * 256),
           kb < nkb && nb < nbN ? ((uint32_t)nb * (uint32_t)nkb + (uint32_t)kb) * 4u : OOB, rsw, 0u);
    }
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
  constexpr int WAIT_VM_STEP = DMA_PER_STEP | (7 << 4) | (15 << 8);  // all but the last step's DMAs landed
  static_assert(DMA_PER_STEP < 16, "vmcnt immediate");
  const float* lsw = reinterpret_cast<const float*>(lds + SW_OFF) + (wn * WN / 128) * MAX_KB;
#pragma unroll
  for (int k = 0; k < NSTAGE - 1; ++k) issue(k);
  if constexpr (NSTAGE > 2)
    __builtin_amdgcn_s_waitcnt(WAIT_VM_STEP);
  else
    __builtin_amdgcn_s_waitcnt(WAIT_VM0);
  __syncthreads();
  // Software pipeline over fragment pairs: the MFMAs of pair q run while the
  // VALU adds pair q - 1's scaled block sum into its accumulator; the last
  // pair of a step is added at the start of the next step, under the latency
  // of that step's first fragment reads.  A-fragments of row i + 1 are read
  // while row i's pairs run (two buffers), B-fragments once per step.
  f32x16 plast = f32x16{};
  float slast = 0.f;
  for (int kt = 0; kt < nkb; ++kt) {
    // stage (kt + NSTAGE - 1) % NSTAGE was last read in step kt - 1, before the barrier that ended it
    issue(kt + NSTAGE - 1);
    const int sidx = kt % NSTAGE;
    const uint8_t* sa_ = lds + sidx * STAGE;
    const uint8_t* sb_ = sa_ + A_STAGE;
    // A fragments: two buffers (row i + 1 read while row i runs) with one wave
    // per SIMD; one buffer (row i + 1 read after row i's last MFMA) with two,
    // whose registers are half as many and whose other wave covers the wait.
    constexpr int FAB = WAVES > 4 ? 1 : 2;
    i32x8 fb0[FJ], fb1[FJ], fa0[FAB], fa1[FAB];
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
      fb0[j] = frag(sb_, b_row + j * 32, 0);
      fb1[j] = frag(sb_, b_row + j * 32, 1);
    }
    fa0[0] = frag(sa_, a_row, 0);
    fa1[0] = frag(sa_, a_row, 1);
    const f32x4 sav = *reinterpret_cast<const f32x4*>(lds + SA_OFF + sidx * BM * 4 + (wm * 128 + 4 * (lane & 31)) * 4);
    const float swv = lsw[kt];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[FI - 1][FJ - 1][e] = __builtin_fmaf(plast[e], slast, acc[FI - 1][FJ - 1][e]);
    float s[FI];
#pragma unroll
    for (int i = 0; i < FI; ++i) s[i] = sav[i] * swv;
    f32x16 pprev = f32x16{};
#pragma unroll
    for (int i = 0; i < FI; ++i) {
      if (FAB == 2 && i + 1 < FI) {
        fa0[(i + 1) % FAB] = frag(sa_, a_row + (i + 1) * 32, 0);
        fa1[(i + 1) % FAB] = frag(sa_, a_row + (i + 1) * 32, 1);
      }
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
        // transposed product (W^T fragment first): a lane holds 4 consecutive columns
        f32x16 p = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb0[j], fa0[i % FAB], f32x16{}, 0, 0, 0, 0, 0, 0);
        p = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb1[j], fa1[i % FAB], p, 0, 0, 0, 0, 0, 0);
        const int q = i * FJ + j;
        if (q > 0) {
          const int pi = (q - 1) / FJ, pj = (q - 1) % FJ;
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[pi][pj][e] = __builtin_fmaf(pprev[e], s[pi], acc[pi][pj][e]);
        }
        pprev = p;
      }
      if (FAB == 1 && i + 1 < FI) {
        fa0[0] = frag(sa_, a_row + (i + 1) * 32, 0);
        fa1[0] = frag(sa_, a_row + (i + 1) * 32, 1);
      }
    }
    // Issue order of the step (one scheduling region): pair q's two MFMAs with
    // pair q - 1's 16 FMAs between and after them (the matrix pipe runs pair q
    // while the VALU adds pair q - 1), and the next A row's fragment reads
    // (4 LDS reads) beside the first MFMA of each row.  At most two block sums
    // are live at a time.
#pragma unroll
    for (int q = 0; q < FI * FJ; ++q) {
      const bool next_row = q / FJ + 1 < FI;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                      // MFMA, first k half
      if (FAB == 2 && q % FJ == 0 && next_row) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // next row's reads
      if (q > 0) __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);          // FMAs of pair q - 1
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                      // MFMA, second k half
      if (FAB == 1 && q % FJ == FJ - 1 && next_row) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
      if (q > 0) __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
    }
    plast = pprev;
    slast = s[FI - 1];
    // stage kt + 1 must land before the barrier that hands it to the next step
    // (with three stages the DMAs of step kt + 2, issued after it, may still be in flight)
    if constexpr (NSTAGE > 2)
      __builtin_amdgcn_s_waitcnt(WAIT_VM_STEP);
    else
      __builtin_amdgcn_s_waitcnt(WAIT_VM0);
    __syncthreads();
  }
  __builtin_amdgcn_s_waitcnt(WAIT_VM0);  // the DMAs issued past the end
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[FI - 1][FJ - 1][e] = __builtin_fmaf(plast[e], slast, acc[FI - 1][FJ - 1][e]);

  // Epilogue: element 4g + e of fragment (i, j) is row i*32 + lane%32, column
  // j*32 + g*8 + (lane/32)*4 + e of the wave tile.  One RNE rounding to bf16 by
  // the hardware converter; the tile is staged in LDS (the operand stages are
  // free now) and stored as 16-byte row chunks, so every HBM write covers whole
  // lines (stored straight from the registers, 8 bytes per lane, the writes
  // counted 2x the output's bytes).
  constexpr int C_STRIDE = BN + 8;  // bf16 per staged row (16-byte pad)
  static_assert((size_t)BM * C_STRIDE * 2 <= C::LDS_BYTES, "staged output tile fits in LDS");
  __syncthreads();  // every wave is done with the operand stages
  uint16_t* ct = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int row = a_row + i * 32;
        const int col = wn * WN + j * 32 + g * 8 + (lane >> 5) * 4;
        u32x2 v;
        v[0] = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                                                (f32x2v{acc[i][j][4 * g], acc[i][j][4 * g + 1]}), bf16x2v));
        v[1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                                                (f32x2v{acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]}), bf16x2v));
        *reinterpret_cast<u32x2*>(ct + row * C_STRIDE + col) = v;
      }
  __syncthreads();
  const int rows = min(BM, M - m0), cols = min(BN, N - n0);
  for (int idx = t; idx < BM * (BN / 8); idx += C::THREADS) {
    const int row = idx / (BN / 8), ch = idx % (BN / 8);
    if (row < rows && ch * 8 < cols) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(ct + row * C_STRIDE + ch * 8);
      *reinterpret_cast<u32x4*>(Y + (int64_t)(m0 + row) * N + n0 + ch * 8) = v;
    }
  }
}

// ------------------------------------------------------------------ activation quantiser

// One 16-lane group per 128-element block of a row (a lane holds 8 halfs),
// IT blocks per group: item i of workgroup b covers blocks 16 (IT b + i) ..
// + 15, so each item's 16 groups read 4 KiB of consecutive blocks (the blocks
// of a row are consecutive), and all IT loads of a lane are issued before the
// first reduction.
// Maximum over the 16 lanes of a DPP row (a lane group): rotations by 8, 4, 2
// and 1 within the row, VALU only.
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false));  // row_ror:8
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xF, 0xF, false));  // row_ror:4
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x122, 0xF, 0xF, false));  // row_ror:2
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x121, 0xF, 0xF, false));  // row_ror:1
  return v;
}

// The block count M * K / 128 is below 2^23 (A < 2 GiB), so block ids and
// their row / block split fit 32-bit arithmetic.
template <int IT>
__global__ void __launch_bounds__(256) fp8_quant_blocks(const u32x4* __restrict__ A, u32x2* __restrict__ Aq,
                                                        float* __restrict__ sa_out, uint32_t M, uint32_t nkb) {
  const uint32_t sub = threadIdx.x & 15, grp = threadIdx.x >> 4;
  const uint32_t total = M * nkb;
  const buf_rsrc_t rs = buf_rsrc(A, total * 256u);
  u32x4 x[IT];
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const uint32_t blk = (blockIdx.x * IT + i) * 16u + grp;  // global block id = m * nkb + kb
    x[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, blk < total ? (blk * 16u + sub) * 16u : BUF_OOB, 0, 2 /* nt */);
  }
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const uint32_t blk = (blockIdx.x * IT + i) * 16u + grp;
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t a = x[i][j] & 0x7FFF7FFFu;
      m = max(m, max(a & 0xFFFFu, a >> 16));
    }
    m = row16_max_u32(m);
    const float amax = (float)__builtin_bit_cast(_Float16, (uint16_t)m);
    const float s = amax / 448.0f;
    const float y = 1.0f / s;
    if (blk < total) {
      const uint32_t row = blk / nkb, kb = blk - row * nkb;
      if (sub == 0) sa_out[kb * M + row] = s;
      Aq[blk * 16u + sub] = quantize_chunk(x[i], s, y, m);
    }
  }
}

template <int BN, int WAVES, int NSTAGE>
tb_status launch_block(const uint8_t* Aq, const uint8_t* WqT, const float* sa, const float* sw, uint16_t* Y,
                       int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  typedef Cfg<BN, WAVES, NSTAGE> C;
  auto kern = &fp8_block_gemm<BN, WAVES, NSTAGE>;
  if (tb_status st = tb::reserve_lds(reinterpret_cast<const void*>(kern), C::LDS_BYTES, "tb_fp8_block_gemm"))
    return st;
  const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
  hipLaunchKernelGGL(kern, dim3(tiles_m * tiles_n), dim3(C::THREADS), C::LDS_BYTES, stream, Aq, WqT, sa, sw, Y, (int)M,
                     (int)N, (int)K, tiles_m, tiles_n);
  return tb::launch_status("tb_fp8_block_gemm");
}

}  // namespace fp8blk
}  // namespace tb

// The launched configuration: 256 x 256 tiles on eight wavefronts (two per
// SIMD), two stages.  Measured at 8192^3 (same box, bit-identical outputs):
// 256 x 128 on four wavefronts with three stages 722 us, this 561-568 us.
namespace {
constexpr int kLaunchBN = 256, kLaunchWaves = 8, kLaunchStages = 2;
// 128-element blocks per lane group of the quantiser: two (34.6 us at 8192^2,
// against 41.3 us with one)
constexpr int kQuantBlocksPerGroup = 2;
}  // namespace

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
  constexpr int IT = kQuantBlocksPerGroup;
  hipLaunchKernelGGL(tb::fp8blk::fp8_quant_blocks<IT>, dim3((unsigned)((blocks + 16 * IT - 1) / (16 * IT))), dim3(256),
                     0, stream, reinterpret_cast<const tb::u32x4*>(A), reinterpret_cast<tb::u32x2*>(Aq), sa,
                     (uint32_t)M, (uint32_t)(K / 128));
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
  TB_CHECK_ALIGN(Y, 16, "Y");
  return launch_block<kLaunchBN, kLaunchWaves, kLaunchStages>(Aq, WqT, sa, sw, Y, M, N, K, stream);
}
