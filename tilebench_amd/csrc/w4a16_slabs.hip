// W4A16 decode (M <= 16) over a slab-contiguous copy of the int4 weights.
//
// The split-K decode in w4a16_gemm.hip reads W in its packed [K, N/2] layout,
// where a block's columns are a strip of every row; to keep every CU streaming
// it splits K over several blocks per column slab and pays a cross-block
// reduction (three round trips to the device coherence point after the last
// block's K loop).  Here the weights are first copied, once per weight tensor,
// into a layout where the 64 columns of a slab are one contiguous run of
// K * 32 bytes, so one block per slab streams its whole K range at the full
// per-CU rate and reduces across its own wavefronts in LDS: no split-K, no
// hand-off between blocks.
//
// Slab layout (tb_w4a16_repack_slabs): slab s holds columns 64 s .. 64 s + 63;
// its unit u (K rows 32 u .. 32 u + 31) is 1 KiB: 64 lanes x 16 bytes, lane l's
// 16 bytes being four 32-bit words, word b holding the 8 codes of column
// 64 s + 16 b + (l % 16) at rows 32 u + 8 (l / 16) + i, i = 0..7, code i at bit
// (i % 2) * 16 + (i / 2) * 4.  That is the lane's B fragment of
// v_mfma_f32_16x16x32_f16 for the 16-column block b: the pairs (i, i + 1) for
// i = 0 and 4 sit in bits 3:0 and 19:16 of the word (read as 1024 + q under the
// 0x64 exponent), those for i = 2 and 6 in bits 7:4 and 23:20 (read as 64 + q
// under 0x54, whose mantissa unit is 1/16), the upper four after one shift by
// 8: five VALU instructions per 8 weights.
//
// Decode (tb_w4a16_gemm_slabs): block s = slab s, 16 wavefronts; wavefront w
// takes units 8 w .. (K / 512 units each), loaded through buffer resources
// (rows of A past M read zeros) four units ahead; the slab's 64 scales and
// zero-points of a group are one load each per wavefront (lane c: column c),
// handed to the lanes that use them by ds_bpermute.  The MFMAs take
// the codes (c0 + q: c0 = 1024 for rows i in {0, 1, 4, 5} of each 8, 64 for
// {2, 3, 6, 7}); per group of G rows the scale and zero-point enter once in
// fp32: sum_k a (q - z) s = s (sum_k a (c0 + q) - 1024 A1 - 64 A2 - z (A1 + A2)),
// A1 and A2 the sums of a over the two row classes, from two more MFMAs against
// ones.  Weights are therefore not rounded to fp16 before the product (as in
// the split-K decode); the 16 wavefront partials are summed in LDS in a fixed
// order, so results are reproducible bit for bit.
#include "tb_common.h"

#pragma clang fp contract(off)

namespace tb {
namespace slabs {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int COLS = 64, THREADS = 1024, WAVES = 16, UNIT = 32, PSTRIDE = COLS + 4;

__device__ __forceinline__ u32x4 ld16(buf_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// One thread per output word: word b of lane l of unit u of slab s.
__global__ void __launch_bounds__(256) slab_repack(const uint8_t* __restrict__ W, uint32_t* __restrict__ Wr, int K,
                                                   int N) {
  const int64_t words = (int64_t)K * N / 8;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= words) return;
  const int b = (int)(t & 3), l = (int)((t >> 2) & 63);
  const int64_t su = t >> 8;  // slab * (K / 32) + unit
  const int units = K / UNIT;
  const int s = (int)(su / units), u = (int)(su % units);
  const int col = s * COLS + b * 16 + (l & 15);
  const int r0 = u * UNIT + (l >> 4) * 8;
  const int half_n = N >> 1;
  uint32_t w = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t q = (W[(int64_t)(r0 + i) * half_n + (col >> 1)] >> (4 * (col & 1))) & 15u;
    w |= q << ((i & 1) * 16 + (i >> 1) * 4);
  }
  Wr[t] = w;
}

// UPW = K / 512 units per wavefront, UPG = G / 32 units per group (both
// compile-time, so no load sits behind a condition the compiler could sink it
// into).
template <int UPW, int UPG>
__global__ void __launch_bounds__(THREADS) slab_decode(const _Float16* __restrict__ A, const uint32_t* __restrict__ Wr,
                                                       const _Float16* __restrict__ S, const uint8_t* __restrict__ Z,
                                                       _Float16* __restrict__ Y, int M, int N, int K, int group) {
  __shared__ float part[WAVES][16 * PSTRIDE];
  const int s = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int MAXU = UPW, upw = UPW, upg = UPG;
  const int units = K / UNIT;
  const int u0 = wave * upw;
  const int arow = lane & 15;

  const buf_rsrc_t rw = buf_rsrc(Wr + (int64_t)s * units * 256, (uint32_t)units * 1024u);
  const buf_rsrc_t ra = buf_rsrc(A, (uint32_t)M * (uint32_t)K * 2u);
  const buf_rsrc_t rs = buf_rsrc(S, (uint32_t)(K / group) * (uint32_t)N * 2u);
  const buf_rsrc_t rz = buf_rsrc(Z, (uint32_t)(K / group) * (uint32_t)(N >> 1));
  const uint32_t a_lane = arow < M ? ((uint32_t)arow * (uint32_t)K + (uint32_t)(lane >> 4) * 8u) * 2u : BUF_OOB;

  // The group scales and zero-points of the wavefront's units first (so the
  // folds never wait on a load issued after the weights), one load of each
  // per group: lane l holds column l's scale and zero-point byte (the lanes
  // that use them get them by ds_bpermute at the group's first unit); then
  // the units, DEPTH in flight: unit i + DEPTH is issued once unit i has been
  // consumed.
  constexpr int MAXG = UPW / UPG;  // groups per wavefront
  uint32_t s_all[MAXG], z_all[MAXG];
#pragma unroll
  for (int j = 0; j < MAXG; ++j) {
    const uint32_t g = (uint32_t)(u0 / upg + j);
    const uint32_t col = (uint32_t)(s * COLS + lane);
    s_all[j] = __builtin_amdgcn_raw_buffer_load_b16(rs, (g * (uint32_t)N + col) * 2u, 0, 0);
    z_all[j] = __builtin_amdgcn_raw_buffer_load_b8(rz, g * (uint32_t)(N >> 1) + (col >> 1), 0, 0);
  }
  constexpr int DEPTH = 4;  // measured: 2 and 8 units ahead 3 % and 1 % slower
  u32x4 wv[MAXU], av[MAXU];
  auto issue = [&](int i) {
    const uint32_t u = (uint32_t)(u0 + i);
    wv[i] = ld16(rw, (u * 64u + (uint32_t)lane) * 16u);
    av[i] = ld16(ra, a_lane + u * UNIT * 2u);
  };
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < DEPTH && i < MAXU; ++i) {
    issue(i);
    __builtin_amdgcn_sched_barrier(0);  // in unit order: the first unit's wait covers only its own loads
  }

  const h8 ones1 = __builtin_bit_cast(h8, u32x4{0x3C003C00u, 0u, 0x3C003C00u, 0u});
  const h8 ones2 = __builtin_bit_cast(h8, u32x4{0u, 0x3C003C00u, 0u, 0x3C003C00u});
  const f32x4v zero{};
  f32x4v acc[4] = {zero, zero, zero, zero};
  f32x4v tmp[4], a1, a2;
  uint32_t sz[4];  // the group's scale (bits 15:0) and zero-point (bits 19:16) of column 16 b + lane % 16
#pragma unroll
  for (int i = 0; i < MAXU; ++i) {
    const bool first = i % upg == 0;
    const h8 af = __builtin_bit_cast(h8, av[i]);
    const u32x4 wi = wv[i];
    if (first) {
      // column c's scale and zero-point nibble (column c = 64 s + c: nibble c % 2) from lane c
      const uint32_t packed = (s_all[i / upg] & 0xFFFFu) | (((z_all[i / upg] >> (4 * (lane & 1))) & 15u) << 16);
#pragma unroll
      for (int b = 0; b < 4; ++b) sz[b] = (uint32_t)__builtin_amdgcn_ds_bpermute((b * 16 + (lane & 15)) * 4, (int)packed);
    }
    // units in pairs: the next two units' loads go out, then both units' work
    // in one scheduling region (measured at M = 16: 9.55 -> 9.24 us)
    if (i % 2 == 0) {
      if (i + DEPTH < MAXU) issue(i + DEPTH);
      if (i + 1 + DEPTH < MAXU) issue(i + 1 + DEPTH);
      __builtin_amdgcn_sched_barrier(0);
    }
    a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, ones1, first ? zero : a1, 0, 0, 0);
    a2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, ones2, first ? zero : a2, 0, 0, 0);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t w = wi[b], w8 = w >> 8;
      const u32x4 bf = {(w & 0x000F000Fu) | 0x64006400u, (w & 0x00F000F0u) | 0x54005400u,
                        (w8 & 0x000F000Fu) | 0x64006400u, (w8 & 0x00F000F0u) | 0x54005400u};
      tmp[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, __builtin_bit_cast(h8, bf), first ? zero : tmp[b], 0, 0, 0);
    }
    if (i % upg == upg - 1) {
      // fold of the group: s (sum a (c0 + q) - 1024 A1 - 64 A2 - z (A1 + A2)) for column 16 b + lane % 16
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const float sf = (float)__builtin_bit_cast(_Float16, (uint16_t)(sz[b] & 0xFFFFu));
        const float zf = (float)(sz[b] >> 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float c = 1024.f * a1[e] + 64.f * a2[e];
          acc[b][e] = __builtin_fmaf(sf, (tmp[b][e] - c) - zf * (a1[e] + a2[e]), acc[b][e]);
        }
      }
    }
  }

  // acc[b][e]: row 4 (lane / 16) + e, column 16 b + lane % 16 of the slab;
  // rows below M only (the lane's rows are 4 (lane / 16) .. +3): M = 1 7.36 -> 7.20 us
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (4 * (lane >> 4) + e < M)
#pragma unroll
      for (int b = 0; b < 4; ++b) part[wave][(4 * (lane >> 4) + e) * PSTRIDE + b * 16 + (lane & 15)] = acc[b][e];
  __syncthreads();
  const int row = threadIdx.x / COLS, col = threadIdx.x % COLS;
  if (row < M) {
    float sum = part[0][row * PSTRIDE + col];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) sum += part[w][row * PSTRIDE + col];
    Y[(int64_t)row * N + s * COLS + col] = (_Float16)sum;
  }
}

}  // namespace slabs
}  // namespace tb

extern "C" {

tb_status tb_w4a16_repack_slabs(const uint8_t* W, uint8_t* Wr, int64_t K, int64_t N, hipStream_t stream) {
  TB_CHECK_ARG(W && Wr, "tb_w4a16_repack_slabs: null pointer");
  TB_CHECK_ARG(K > 0 && N > 0 && K % 32 == 0 && N % 64 == 0,
               "tb_w4a16_repack_slabs: need K %% 32 == 0 and N %% 64 == 0 (K=%lld N=%lld)", (long long)K, (long long)N);
  TB_CHECK_ARG(K * N / 2 < (1ll << 31), "tb_w4a16_repack_slabs: weights must be smaller than 2 GiB");
  TB_CHECK_ALIGN(Wr, 16, "Wr");
  const int64_t words = K * N / 8;
  hipLaunchKernelGGL(tb::slabs::slab_repack, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, stream, W,
                     reinterpret_cast<uint32_t*>(Wr), (int)K, (int)N);
  return tb::launch_status("tb_w4a16_repack_slabs");
}

tb_status tb_w4a16_gemm_slabs(const uint16_t* A, const uint8_t* Wr, const uint16_t* scales, const uint8_t* zeros,
                              uint16_t* Y, int64_t M, int64_t N, int64_t K, int64_t group, hipStream_t stream) {
  using namespace tb::slabs;
  TB_CHECK_ARG(A && Wr && scales && zeros && Y, "tb_w4a16_gemm_slabs: null pointer");
  TB_CHECK_ARG(M >= 1 && M <= 16, "tb_w4a16_gemm_slabs: needs 1 <= M <= 16 (M=%lld)", (long long)M);
  TB_CHECK_ARG(N > 0 && N % COLS == 0, "tb_w4a16_gemm_slabs: N must be a positive multiple of %d (N=%lld)", COLS,
               (long long)N);
  TB_CHECK_ARG((group == 64 || group == 128) && (K == 1024 || K == 2048 || K == 4096) && K % (WAVES * group) == 0,
               "tb_w4a16_gemm_slabs: needs G in {64, 128}, K in {1024, 2048, 4096} and K %% (16 G) == 0 "
               "(K=%lld group=%lld)", (long long)K, (long long)group);
  TB_CHECK_ARG(M * K * 2 < (1ll << 31) && K * N / 2 < (1ll << 31) && (K / group) * N * 2 < (1ll << 31),
               "tb_w4a16_gemm_slabs: operands must be smaller than 2 GiB");
  TB_CHECK_ALIGN(A, 16, "A");
  TB_CHECK_ALIGN(Wr, 16, "Wr");
  const int upw = (int)(K / (WAVES * UNIT)), upg = (int)(group / UNIT);
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)(N / COLS)), dim3(THREADS), 0, stream, reinterpret_cast<const _Float16*>(A),
                       reinterpret_cast<const uint32_t*>(Wr), reinterpret_cast<const _Float16*>(scales), zeros,
                       reinterpret_cast<_Float16*>(Y), (int)M, (int)N, (int)K, (int)group);
  };
  if (upw == 8 && upg == 4)
    launch(slab_decode<8, 4>);
  else if (upw == 8 && upg == 2)
    launch(slab_decode<8, 2>);
  else if (upw == 4 && upg == 4)
    launch(slab_decode<4, 4>);
  else if (upw == 4 && upg == 2)
    launch(slab_decode<4, 2>);
  else
    launch(slab_decode<2, 2>);
  return tb::launch_status("tb_w4a16_gemm_slabs");
}

}  // extern "C"
