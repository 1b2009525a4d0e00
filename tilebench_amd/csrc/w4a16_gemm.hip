// W4A16 GEMM: Y[M, N] = fp16(A[M, K] @ dequant(W)[K, N]), fp32 accumulation.
//
// A is fp16 row-major; W is int4 in the N-packed, low-nibble-first layout with
// group-wise fp16 scales and int4 zero-points along K (see include/tbhip.h).
//
// Prefill kernel (MFMA-bound for large M): 256 x 256 output tile per
// 256-thread block, four wavefronts in a 2 x 2 arrangement each owning a
// 128 x 128 sub-tile (16 v_mfma_f32_32x32x16_f16 accumulators = 256 fp32 per
// lane), K advanced 64 at a time through a two-stage LDS pipeline:
//
//   global -> registers : the A tile (256 x 64 fp16, eight 16-byte loads per
//                         thread) and the packed W tile (64 x 256 int4, eight
//                         4-byte row loads per thread: 8 rows x 8 columns) for
//                         step i+1 are issued before the MFMAs of step i;
//   dequantise          : each thread turns its 8 x 8 int4 block into fp16 once
//                         per block ((1024 + q) via the 0x6400 magic number,
//                         exact zero-point subtraction, one RNE multiply by the
//                         scale: bit-identical to the standalone dequantiser) and
//                         transposes it with byte permutes so that every column
//                         holds 8 consecutive k;
//   LDS                 : A as [256][64] and W^T as [256][64] fp16, 16-byte chunks
//                         XOR-swizzled by (row & 7) so the fragment reads of a
//                         wavefront spread over all banks;
//   MFMA                : per k16 step each wavefront reads 4 A and 4 B fragments
//                         (one ds_read_b128 per lane each) and issues 16 MFMAs.
//
// Tiles are numbered XCD-aware: consecutive hardware block ids land on
// different XCDs, so block ids are first regrouped so that each XCD owns a
// contiguous run of tiles, and runs are ordered in groups of 4 tile rows, so
// the blocks resident on one XCD share A rows and W columns in its L2.
#include "tb_common.h"

#include <algorithm>

#pragma clang fp contract(off)

namespace tb {
namespace w4a16 {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 256, BN = 256, BK = 64, THREADS = 256;
constexpr int GROUP_M = 4;  // tile rows per ordering group
constexpr int STAGE_HALFS = (BM + BN) * BK;
constexpr size_t LDS_BYTES = 2 * STAGE_HALFS * sizeof(_Float16);  // 128 KiB

__device__ __forceinline__ int swz(int row, int chunk) { return (row * 8 + (chunk ^ (row & 7))) * 8; }

// (1024 + q) half2 pairs of one packed dword: columns (0,1), (2,3), (4,5), (6,7).
__device__ __forceinline__ void unpack8(uint32_t w, f16x2 (&h)[4]) {
  const uint32_t even = w & 0x0F0F0F0Fu;
  const uint32_t odd = (w >> 4) & 0x0F0F0F0Fu;
  h[0] = magic_h2(perm(odd, even, 0x0C040C00u));
  h[1] = magic_h2(perm(odd, even, 0x0C050C01u));
  h[2] = magic_h2(perm(odd, even, 0x0C060C02u));
  h[3] = magic_h2(perm(odd, even, 0x0C070C03u));
}

struct Tile {
  int m0, n0;
};

__device__ __forceinline__ Tile tile_of_block(int tiles_m, int tiles_n) {
  const int nb = tiles_m * tiles_n;
  int bid = blockIdx.x;
  if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);  // contiguous run per XCD
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

struct Prefetch {
  u32x4 a[8];
  uint32_t w[8];
  u32x4 s;
  uint32_t z;
};

__device__ __forceinline__ void load_tile(Prefetch& p, const _Float16* __restrict__ A, const uint8_t* __restrict__ W,
                                          const _Float16* __restrict__ S, const uint8_t* __restrict__ Z, int M,
                                          int N, int K, int group, int m0, int n0, int k0) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int id = i * THREADS + t, row = id >> 3, c = id & 7;
    const int m = m0 + row;
    if (m < M) p.a[i] = *reinterpret_cast<const u32x4*>(A + (int64_t)m * K + k0 + c * 8);
    else p.a[i] = u32x4{0u, 0u, 0u, 0u};
  }
  const int cg = t & 31, kg = t >> 5;
  const int n = n0 + cg * 8;
  if (n < N) {
    const int64_t half_n = N >> 1;
#pragma unroll
    for (int r = 0; r < 8; ++r)
      p.w[r] = *reinterpret_cast<const uint32_t*>(W + (int64_t)(k0 + kg * 8 + r) * half_n + (n >> 1));
    const int g = k0 / group;
    p.s = *reinterpret_cast<const u32x4*>(S + (int64_t)g * N + n);
    p.z = *reinterpret_cast<const uint32_t*>(Z + (int64_t)g * half_n + (n >> 1));
  } else {
#pragma unroll
    for (int r = 0; r < 8; ++r) p.w[r] = 0u;
    p.s = u32x4{0u, 0u, 0u, 0u};
    p.z = 0u;
  }
}

__device__ __forceinline__ void store_tile(const Prefetch& p, _Float16* __restrict__ lds) {
  const int t = threadIdx.x;
  _Float16* la = lds;
  _Float16* lb = lds + BM * BK;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int id = i * THREADS + t, row = id >> 3, c = id & 7;
    *reinterpret_cast<u32x4*>(la + swz(row, c)) = p.a[i];
  }
  // Dequantise the 8 x 8 block: rows kg*8 + r, columns cg*8 + 0..7.
  const int cg = t & 31, kg = t >> 5;
  f16x2 zh[4], sh[4];
  unpack8(p.z, zh);
#pragma unroll
  for (int j = 0; j < 4; ++j) sh[j] = as_h2(p.s[j]);
  uint32_t d[8][4];  // d[r][j] = half2(col 2j, col 2j+1) of row r
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    f16x2 h[4];
    unpack8(p.w[r], h);
#pragma unroll
    for (int j = 0; j < 4; ++j) d[r][j] = as_u32((h[j] - zh[j]) * sh[j]);
  }
  // 2 x 2 half transposes: column 2j+e gets rows (2p, 2p+1) in one dword.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t sel = e ? 0x07060302u : 0x05040100u;
      u32x4 col;
#pragma unroll
      for (int q = 0; q < 4; ++q) col[q] = perm(d[2 * q + 1][j], d[2 * q][j], sel);
      const int nrow = cg * 8 + 2 * j + e;
      *reinterpret_cast<u32x4*>(lb + swz(nrow, kg)) = col;
    }
  }
}

__global__ void __launch_bounds__(THREADS, 1)
    w4a16_prefill(const _Float16* __restrict__ A, const uint8_t* __restrict__ W, const _Float16* __restrict__ S,
                  const uint8_t* __restrict__ Z, _Float16* __restrict__ Y, int M, int N, int K, int group,
                  int tiles_m, int tiles_n) {
  extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
  const Tile tile = tile_of_block(tiles_m, tiles_n);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  Prefetch pf;
  load_tile(pf, A, W, S, Z, M, N, K, group, tile.m0, tile.n0, 0);
  store_tile(pf, lds);
  __syncthreads();

  const int nk = K / BK;
  for (int it = 0; it < nk; ++it) {
    const bool more = it + 1 < nk;
    if (more) load_tile(pf, A, W, S, Z, M, N, K, group, tile.m0, tile.n0, (it + 1) * BK);
    const _Float16* la = lds + (it & 1) * STAGE_HALFS;
    const _Float16* lb = la + BM * BK;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int chunk = ks * 2 + (lane >> 5);
      h8 af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = wm * 128 + i * 32 + (lane & 31);
        af[i] = *reinterpret_cast<const h8*>(la + swz(row, chunk));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = wn * 128 + j * 32 + (lane & 31);
        bf[j] = *reinterpret_cast<const h8*>(lb + swz(col, chunk));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (more) store_tile(pf, lds + ((it + 1) & 1) * STAGE_HALFS);
    __syncthreads();
  }

  // Epilogue: accumulator element e of fragment (i, j) is row
  // i*32 + (e/4)*8 + (lane/32)*4 + e%4, column j*32 + lane%32 of the wave tile.
  const int col_base = tile.n0 + wn * 128 + (lane & 31);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = tile.m0 + wm * 128 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
      if (m < M) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int n = col_base + j * 32;
          if (n < N) Y[(int64_t)m * N + n] = (_Float16)acc[i][j][e];
        }
      }
    }
  }
}


// ---------------------------------------------------------------------------
// Decode kernel (M <= 16, HBM-bound on the weights).  A block owns a 128-column
// slab and one of S contiguous K ranges; its four wavefronts take the range's
// 32-row units round-robin.  Per unit a lane loads an 8 x 8 int4 block (eight
// 4-byte row loads, 16 lanes side by side cover 64 contiguous bytes of a row),
// dequantises and transposes it exactly as the prefill kernel does, and feeds
// eight v_mfma_f32_16x16x32_f16 (A rows >= M are zero): fragment j holds
// columns 8c + j, c = lane % 16.  The four wave partials are summed in LDS in
// a fixed order, so results are reproducible bit for bit.
// Across the S blocks of a slab the reduction is a serial split-K: each block
// stores its fp32 partial in the workspace, then bumps the slab's arrival
// counter; the block that arrives last adds the S partials in slot order
// (deterministic), writes fp16 Y and puts the counter back to zero, so the
// workspace is ready for the next call without any clearing.
constexpr int DEC_COLS = 128, DEC_THREADS = 256, DEC_UNIT = 32, DEC_PREFETCH = 4;
// Workspace layout, the same for every shape so that calls of different shapes
// can share one buffer: [DEC_MAX_SLABS int32 arrival counters][fp32 partials].
// Counters are left at zero by every call; partials never overlap them.
constexpr int64_t DEC_MAX_SLABS = 4096;
constexpr int64_t DEC_COUNTER_BYTES = DEC_MAX_SLABS * 4;

typedef _Float16 h8d __attribute__((ext_vector_type(8)));
typedef float f32x4d __attribute__((ext_vector_type(4)));

struct DecUnit {
  uint32_t w[8];
  u32x4 a;
  u32x4 s;
  uint32_t z;
};

__global__ void __launch_bounds__(DEC_THREADS)
    w4a16_decode(const _Float16* __restrict__ A, const uint8_t* __restrict__ W, const _Float16* __restrict__ S,
                 const uint8_t* __restrict__ Z, _Float16* __restrict__ Y, float* __restrict__ partials,
                 int* __restrict__ counters, int M, int N, int K, int group, int splits) {
  __shared__ float part[4][16 * DEC_COLS];  // one partial per wavefront, summed in fixed order
  __shared__ float red[16 * DEC_COLS];
  __shared__ int last_flag;
  const int slab = blockIdx.x / splits, split = blockIdx.x % splits;
  const int n0 = slab * DEC_COLS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, kg = lane >> 4;
  const int n = n0 + c * 8;
  const bool col_ok = n < N;
  const int units = K / DEC_UNIT;
  const int u_begin = (int)((int64_t)units * split / splits), u_end = (int)((int64_t)units * (split + 1) / splits);
  const int64_t half_n = N >> 1;
  const int arow = lane & 15;


  f32x4d acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x4d{};

  auto load_unit = [&](DecUnit& d, int u) {
    const int k = u * DEC_UNIT + kg * 8;
#pragma unroll
    for (int r = 0; r < 8; ++r)
      d.w[r] = col_ok ? __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(W + (int64_t)(k + r) * half_n + (n >> 1)))
                      : 0u;
    d.a = arow < M ? *reinterpret_cast<const u32x4*>(A + (int64_t)arow * K + k) : u32x4{0u, 0u, 0u, 0u};
    const int g = (u * DEC_UNIT) / group;
    d.s = col_ok ? *reinterpret_cast<const u32x4*>(S + (int64_t)g * N + n) : u32x4{0u, 0u, 0u, 0u};
    d.z = col_ok ? *reinterpret_cast<const uint32_t*>(Z + (int64_t)g * half_n + (n >> 1)) : 0u;
  };

  for (int u0 = u_begin + wave; u0 < u_end; u0 += 4 * DEC_PREFETCH) {
    DecUnit d[DEC_PREFETCH];
#pragma unroll
    for (int p = 0; p < DEC_PREFETCH; ++p)
      if (u0 + 4 * p < u_end) load_unit(d[p], u0 + 4 * p);
#pragma unroll
    for (int p = 0; p < DEC_PREFETCH; ++p) {
      const int u = u0 + 4 * p;
      if (u >= u_end) break;
      f16x2 zh[4], sh[4];
      unpack8(d[p].z, zh);
#pragma unroll
      for (int j = 0; j < 4; ++j) sh[j] = as_h2(d[p].s[j]);
      uint32_t dq[8][4];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        f16x2 h[4];
        unpack8(d[p].w[r], h);
#pragma unroll
        for (int j = 0; j < 4; ++j) dq[r][j] = as_u32((h[j] - zh[j]) * sh[j]);
      }
      const h8d af = __builtin_bit_cast(h8d, d[p].a);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const uint32_t sel = e ? 0x07060302u : 0x05040100u;
          u32x4 col;
#pragma unroll
          for (int q = 0; q < 4; ++q) col[q] = perm(dq[2 * q + 1][j], dq[2 * q][j], sel);
          acc[2 * j + e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, __builtin_bit_cast(h8d, col), acc[2 * j + e], 0, 0, 0);
        }
      }
    }
  }
  // Fragment j, element e: row 4 * (lane / 16) + e, column 8 * (lane % 16) + j.
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) part[wave][(4 * kg + e) * DEC_COLS + c * 8 + j] = acc[j][e];
  __syncthreads();
  for (int i = threadIdx.x; i < 16 * DEC_COLS; i += DEC_THREADS)
    red[i] = ((part[0][i] + part[1][i]) + part[2][i]) + part[3][i];
  __syncthreads();

  const int ncols = min(DEC_COLS, N - n0);
  if (splits == 1) {
    for (int i = threadIdx.x; i < M * DEC_COLS; i += DEC_THREADS) {
      const int m = i / DEC_COLS, cc = i % DEC_COLS;
      if (cc < ncols) Y[(int64_t)m * N + n0 + cc] = (_Float16)red[i];
    }
    return;
  }
  // Serial split-K across the slab's blocks.  Every access to the partials and
  // the counters is a device-scope atomic (coherent across the XCDs' L2s), so
  // no cache-wide fence is needed: each thread waits until its partial stores
  // are acknowledged (s_waitcnt 0) before the block's arrival is counted, and
  // the last block reads the partials with device-scope loads.  (A release /
  // acquire fence would write back and invalidate the whole L2 of the XCD in
  // every block.)
  float* mine = partials + ((int64_t)split * M) * N;
  for (int i = threadIdx.x; i < M * DEC_COLS; i += DEC_THREADS) {
    const int m = i / DEC_COLS, cc = i % DEC_COLS;
    if (cc < ncols) __hip_atomic_store(&mine[(int64_t)m * N + n0 + cc], red[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&counters[slab], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = (prev == splits - 1);
  }
  __syncthreads();
  if (!last_flag) return;
  for (int i = threadIdx.x; i < M * DEC_COLS; i += DEC_THREADS) {
    const int m = i / DEC_COLS, cc = i % DEC_COLS;
    if (cc >= ncols) continue;
    float sum = 0.f;
    for (int s2 = 0; s2 < splits; ++s2)
      sum += s2 == split ? red[i]
                         : __hip_atomic_load(&partials[((int64_t)s2 * M + m) * N + n0 + cc], __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
    Y[(int64_t)m * N + n0 + cc] = (_Float16)sum;
  }
  if (threadIdx.x == 0) __hip_atomic_store(&counters[slab], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

inline int decode_splits(int N, int K) {
  const int slabs = (N + DEC_COLS - 1) / DEC_COLS;
  const int units = K / DEC_UNIT;
  int s = (512 + slabs - 1) / slabs;  // aim at ~2 blocks per CU
  s = std::max(1, std::min(s, units / 4));
  return s;
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

extern "C" tb_status tb_w4a16_gemm(const uint16_t* A, const uint8_t* W, const uint16_t* scales, const uint8_t* zeros,
                                   uint16_t* Y, int64_t M, int64_t N, int64_t K, int64_t group, void* workspace,
                                   int64_t workspace_bytes, hipStream_t stream) {
  using namespace tb::w4a16;
  TB_CHECK_ARG(A && W && scales && zeros && Y, "tb_w4a16_gemm: null pointer");
  TB_CHECK_ARG(M > 0 && N > 0 && K > 0 && group > 0, "tb_w4a16_gemm: sizes must be positive");
  TB_CHECK_ARG(M < (1 << 30) && N < (1 << 30) && K < (1 << 30), "tb_w4a16_gemm: sizes too large");
  TB_CHECK_ARG(N % 8 == 0, "tb_w4a16_gemm: N must be a multiple of 8 (got %lld)", (long long)N);
  TB_CHECK_ARG(K % BK == 0 && group % BK == 0 && K % group == 0,
               "tb_w4a16_gemm: need K %% 64 == 0, group %% 64 == 0 and K %% group == 0 (K=%lld group=%lld)",
               (long long)K, (long long)group);
  TB_CHECK_ALIGN(A, 16, "A");
  TB_CHECK_ALIGN(W, 4, "W");
  TB_CHECK_ALIGN(scales, 16, "scales");
  TB_CHECK_ALIGN(zeros, 4, "zeros");
  TB_CHECK_ALIGN(Y, 2, "Y");
  if (M <= 16) {
    int64_t need = 0;
    tb_w4a16_workspace_size(M, N, K, group, &need);
    const int splits = decode_splits((int)N, (int)K);
    if (need > 0) {
      TB_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                   "tb_w4a16_gemm: M=%lld needs a %lld-byte workspace (got %lld)", (long long)M, (long long)need,
                   (long long)workspace_bytes);
      if (!tb::aligned(workspace, 256)) {
        tb::set_error("tb_w4a16_gemm: workspace must be 256-byte aligned");
        return TB_E_ALIGN;
      }
    }
    const int64_t slabs = (N + DEC_COLS - 1) / DEC_COLS;
    TB_CHECK_ARG(splits == 1 || slabs <= DEC_MAX_SLABS, "tb_w4a16_gemm: N=%lld is too wide for the decode kernel",
                 (long long)N);
    int* counters = reinterpret_cast<int*>(workspace);
    float* partials =
        need > 0 ? reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + DEC_COUNTER_BYTES) : nullptr;
    hipLaunchKernelGGL(w4a16_decode, dim3((unsigned)(slabs * splits)), dim3(DEC_THREADS), 0, stream,
                       reinterpret_cast<const _Float16*>(A), W, reinterpret_cast<const _Float16*>(scales), zeros,
                       reinterpret_cast<_Float16*>(Y), partials, counters, (int)M, (int)N, (int)K, (int)group, splits);
    return tb::launch_status("tb_w4a16_gemm(decode)");
  }
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&w4a16_prefill), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)LDS_BYTES) != hipSuccess) {
      tb::set_error("tb_w4a16_gemm: cannot reserve %zu bytes of LDS", LDS_BYTES);
      return TB_E_HIP;
    }
    attr_set = true;
  }
  const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
  hipLaunchKernelGGL(w4a16_prefill, dim3(tiles_m * tiles_n), dim3(THREADS), LDS_BYTES, stream,
                     reinterpret_cast<const _Float16*>(A), W, reinterpret_cast<const _Float16*>(scales), zeros,
                     reinterpret_cast<_Float16*>(Y), (int)M, (int)N, (int)K, (int)group, tiles_m, tiles_n);
  return tb::launch_status("tb_w4a16_gemm");
}
