// MoE layer around the grouped W4A16 GEMM: routing -> sort -> gate/up + SiLU
// -> down -> weighted combine, one launch per step on one stream.
//
//   gating  : tb_moe_topk_gating (top-k of each token's router logits,
//             softmax over the k values), fp32 weights, int32 expert ids;
//   align   : moe_align_kernel, the (token, slot) pairs p = t * topk + j
//             sorted by expert, stable in p, and the expert row offsets;
//   gate_up : moe_gate_up (w4a16_gemm.hip), X rows gathered per pair,
//             fp16(silu(g) * u) written in sorted order;
//   down    : moe_down (w4a16_gemm.hip), scaled by the pair's weight in fp32,
//             stored fp16 at row p of a token-major [pairs, H] buffer;
//   combine : moe_combine_kernel, out[t] = fp16(sum_j fp32(y[t * topk + j]))
//             in slot order, so results are reproducible bit for bit.
//
// The align kernel runs one block per expert.  Every block reads the whole id
// list twice: first counting the pairs of lower experts (its first row) and of
// its own, then compacting its own pairs in list order.  No atomics, and the
// result does not depend on scheduling.
#include "tb_common.h"

namespace tb {
namespace moe {

constexpr int ALIGN_THREADS = 1024, ALIGN_WAVES = ALIGN_THREADS / 64;
constexpr int IDS_PER_LANE = 16;  // ids a lane takes per step: 64 contiguous bytes
constexpr int WAVE_STEP = 64 * IDS_PER_LANE;

// Ids [i0, i0 + 16) of this lane (ids past `end` read as -1): four 16-byte
// loads when the list is 16-byte aligned.
__device__ __forceinline__ void load16(const int* __restrict__ ids, int64_t i0, int64_t end, bool vec,
                                       int (&v)[IDS_PER_LANE]) {
  if (vec && i0 + IDS_PER_LANE <= end) {
#pragma unroll
    for (int u = 0; u < IDS_PER_LANE / 4; ++u) {
      const int4 x = *reinterpret_cast<const int4*>(ids + i0 + 4 * u);
      v[4 * u] = x.x;
      v[4 * u + 1] = x.y;
      v[4 * u + 2] = x.z;
      v[4 * u + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int u = 0; u < IDS_PER_LANE; ++u) v[u] = i0 + u < end ? ids[i0 + u] : -1;
  }
}

// Block e places expert e's pairs.  Wavefront w owns slice w of the id list
// (contiguous, so slice order is list order): it counts the ids of lower
// experts and of expert e in its slice, the block adds the 16 slice counts,
// and each wavefront then compacts its own slice from its slice's base with
// a wave-level prefix sum only.  Every step prefetches the next step's ids.
__global__ void __launch_bounds__(ALIGN_THREADS)
    moe_align_kernel(const int* __restrict__ ids, int64_t pairs, int experts, int* __restrict__ sorted,
                     int* __restrict__ offsets, bool vec) {
  __shared__ int red[2][ALIGN_WAVES];
  const int e = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t slice = (pairs + ALIGN_WAVES * WAVE_STEP - 1) / (ALIGN_WAVES * WAVE_STEP) * WAVE_STEP;
  const int64_t s_begin = min(pairs, slice * wave), s_end = min(pairs, s_begin + slice);

  // pass 1: ids of lower experts and of this one in the slice
  int below = 0, mine = 0;
  {
    int cur[IDS_PER_LANE], nxt[IDS_PER_LANE];
    load16(ids, s_begin + lane * IDS_PER_LANE, s_end, vec, cur);
    for (int64_t b = s_begin; b < s_end; b += WAVE_STEP) {
      if (b + WAVE_STEP < s_end) load16(ids, b + WAVE_STEP + lane * IDS_PER_LANE, s_end, vec, nxt);
#pragma unroll
      for (int u = 0; u < IDS_PER_LANE; ++u) {
        below += (unsigned)cur[u] < (unsigned)e;  // ids outside [0, experts) are routed nowhere
        mine += cur[u] == e;
      }
#pragma unroll
      for (int u = 0; u < IDS_PER_LANE; ++u) cur[u] = nxt[u];
    }
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    below += __shfl_xor(below, d);
    mine += __shfl_xor(mine, d);
  }
  if (lane == 0) {
    red[0][wave] = below;
    red[1][wave] = mine;
  }
  __syncthreads();
  int first = 0, count = 0, before = 0;
#pragma unroll
  for (int w = 0; w < ALIGN_WAVES; ++w) {
    first += red[0][w];
    count += red[1][w];
    before += w < wave ? red[1][w] : 0;
  }
  if (threadIdx.x == 0) {
    offsets[e] = first;
    if (e == experts - 1) offsets[experts] = first + count;
  }
  if (red[1][wave] == 0) return;  // nothing of expert e in this slice (uniform per wavefront)

  // pass 2: stable compaction of the slice
  int pos = first + before;
  int cur[IDS_PER_LANE], nxt[IDS_PER_LANE];
  load16(ids, s_begin + lane * IDS_PER_LANE, s_end, vec, cur);
  for (int64_t b = s_begin; b < s_end; b += WAVE_STEP) {
    if (b + WAVE_STEP < s_end) load16(ids, b + WAVE_STEP + lane * IDS_PER_LANE, s_end, vec, nxt);
    int c = 0;
#pragma unroll
    for (int u = 0; u < IDS_PER_LANE; ++u) c += cur[u] == e;
    int incl = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d);
      if (lane >= d) incl += o;
    }
    int p = pos + incl - c;
    const int64_t i0 = b + lane * IDS_PER_LANE;
#pragma unroll
    for (int u = 0; u < IDS_PER_LANE; ++u)
      if (cur[u] == e) sorted[p++] = (int)(i0 + u);
    pos += __shfl(incl, 63);
#pragma unroll
    for (int u = 0; u < IDS_PER_LANE; ++u) cur[u] = nxt[u];
  }
}

// out[t, c .. c+7] = fp16(sum_j fp32(y[t * topk + j, c .. c+7])), slots with an
// expert id outside [0, experts) skipped.  One 16-byte granule per thread.
// All of a token's ids are loaded first, then all its rows (an unrouted slot
// through an out-of-range offset, reading zeros without memory traffic, and
// skipped in the sum so that results do not depend on it): one round trip
// per thread instead of one per slot.
template <int KMAX>
__global__ void __launch_bounds__(256)
    moe_combine_kernel(const u32x4* __restrict__ y, const int* __restrict__ ids, u32x4* __restrict__ out,
                       int64_t tokens, int topk, int experts, int64_t g_per_row) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= tokens * g_per_row) return;
  const int64_t tok = g / g_per_row, c = g - tok * g_per_row;
  const buf_rsrc_t rid = buf_rsrc(ids + tok * topk, (uint32_t)topk * 4u);
  int id[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j)
    id[j] = (int)__builtin_amdgcn_raw_buffer_load_b32(rid, j < topk ? (uint32_t)j * 4u : BUF_OOB, 0, 0);
  const buf_rsrc_t ry = buf_rsrc(y + tok * topk * g_per_row, (uint32_t)(topk * g_per_row * 16));
  u32x4 v[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    const bool ok = j < topk && (unsigned)id[j] < (unsigned)experts;
    v[j] = __builtin_amdgcn_raw_buffer_load_b128(ry, ok ? (uint32_t)((j * g_per_row + c) * 16) : BUF_OOB, 0,
                                                 2 /* nt */);
  }
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (!(j < topk && (unsigned)id[j] < (unsigned)experts)) continue;  // slot order, unrouted slots skipped
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f16x2 h = as_h2(v[j][q]);
      s[2 * q] += (float)h[0];
      s[2 * q + 1] += (float)h[1];
    }
  }
  u32x4 o;
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = as_u32(f16x2{(_Float16)s[2 * q], (_Float16)s[2 * q + 1]});
  out[g] = o;
}

inline int64_t round256(int64_t b) { return (b + 255) & ~int64_t(255); }

struct Workspace {
  float* w;
  int* ids;
  int* sorted;
  int* offsets;
  uint16_t* act;
  uint16_t* y;
  int64_t bytes;
};

inline Workspace carve(void* base, int64_t tokens, int64_t topk, int64_t experts, int64_t H, int64_t I) {
  const int64_t pairs = tokens * topk;
  Workspace ws{};
  char* p = reinterpret_cast<char*>(base);
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    char* r = p ? p + off : nullptr;
    off += round256(bytes);
    return r;
  };
  ws.w = reinterpret_cast<float*>(take(pairs * 4));
  ws.ids = reinterpret_cast<int*>(take(pairs * 4));
  ws.sorted = reinterpret_cast<int*>(take(pairs * 4));
  ws.offsets = reinterpret_cast<int*>(take((experts + 1) * 4));
  ws.act = reinterpret_cast<uint16_t*>(take(pairs * I * 2));
  ws.y = reinterpret_cast<uint16_t*>(take(pairs * H * 2));
  ws.bytes = off;
  return ws;
}

}  // namespace moe
}  // namespace tb

extern "C" tb_status tb_moe_align(const int32_t* topk_ids, int64_t pairs, int64_t experts, int32_t* sorted_ids,
                                  int32_t* offsets, hipStream_t stream) {
  using namespace tb::moe;
  TB_CHECK_ARG(topk_ids && sorted_ids && offsets, "tb_moe_align: null pointer");
  TB_CHECK_ARG(pairs > 0 && pairs < (1ll << 31), "tb_moe_align: need 0 < pairs < 2^31 (got %lld)", (long long)pairs);
  TB_CHECK_ARG(experts > 0 && experts <= 4096, "tb_moe_align: need 0 < experts <= 4096 (got %lld)",
               (long long)experts);
  TB_CHECK_ALIGN(topk_ids, 4, "topk_ids");
  TB_CHECK_ALIGN(sorted_ids, 4, "sorted_ids");
  TB_CHECK_ALIGN(offsets, 4, "offsets");
  hipLaunchKernelGGL(moe_align_kernel, dim3((unsigned)experts), dim3(ALIGN_THREADS), 0, stream, topk_ids, pairs,
                     (int)experts, sorted_ids, offsets, tb::aligned(topk_ids, 16));
  return tb::launch_status("tb_moe_align");
}

extern "C" tb_status tb_moe_combine(const uint16_t* y, const int32_t* topk_ids, uint16_t* out, int64_t tokens,
                                    int64_t topk, int64_t experts, int64_t H, hipStream_t stream) {
  using namespace tb::moe;
  TB_CHECK_ARG(y && topk_ids && out, "tb_moe_combine: null pointer");
  TB_CHECK_ARG(tokens > 0 && topk > 0 && experts > 0 && H > 0, "tb_moe_combine: sizes must be positive");
  TB_CHECK_ARG(H % 8 == 0, "tb_moe_combine: H must be a multiple of 8 (got %lld)", (long long)H);
  TB_CHECK_ARG(tokens * topk < (1ll << 31), "tb_moe_combine: tokens * topk must be < 2^31");
  TB_CHECK_ARG(topk <= 32, "tb_moe_combine: topk must be at most 32 (got %lld)", (long long)topk);
  TB_CHECK_ARG(topk * H * 2 < (1ll << 31), "tb_moe_combine: a token's topk rows must be < 2 GiB");
  TB_CHECK_ALIGN(y, 16, "y");
  TB_CHECK_ALIGN(out, 16, "out");
  TB_CHECK_ALIGN(topk_ids, 4, "topk_ids");
  const int64_t g_per_row = H / 8, granules = tokens * g_per_row;
  const int64_t blocks = (granules + 255) / 256;
  TB_CHECK_ARG(blocks < (1ll << 31), "tb_moe_combine: problem too large");
  auto* yv = reinterpret_cast<const tb::u32x4*>(y);
  auto* ov = reinterpret_cast<tb::u32x4*>(out);
  if (topk <= 8)
    hipLaunchKernelGGL(moe_combine_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, stream, yv, topk_ids, ov, tokens,
                       (int)topk, (int)experts, g_per_row);
  else
    hipLaunchKernelGGL(moe_combine_kernel<32>, dim3((unsigned)blocks), dim3(256), 0, stream, yv, topk_ids, ov, tokens,
                       (int)topk, (int)experts, g_per_row);
  return tb::launch_status("tb_moe_combine");
}

extern "C" tb_status tb_fused_moe_w4a16_workspace_size(int64_t tokens, int64_t topk, int64_t experts, int64_t H,
                                                       int64_t I, int64_t* bytes) {
  TB_CHECK_ARG(bytes != nullptr, "tb_fused_moe_w4a16_workspace_size: null output");
  TB_CHECK_ARG(tokens > 0 && topk > 0 && experts > 0 && H > 0 && I > 0,
               "tb_fused_moe_w4a16_workspace_size: sizes must be positive");
  *bytes = tb::moe::carve(nullptr, tokens, topk, experts, H, I).bytes;
  return TB_OK;
}

extern "C" tb_status tb_moe_topk_gating(const void* logits, void* weights, int32_t* indices, int64_t M, int64_t E,
                                        int64_t k, int dtype, hipStream_t stream);
extern "C" tb_status tb_moe_w4a16_gate_up(const uint16_t* X, const int32_t* sorted_ids, const int32_t* offsets,
                                          const uint8_t* W13, const uint16_t* S13, const uint8_t* Z13, uint16_t* act,
                                          int64_t tokens, int64_t topk, int64_t experts, int64_t H, int64_t I,
                                          int64_t group, hipStream_t stream);
extern "C" tb_status tb_moe_w4a16_down(const uint16_t* act, const int32_t* sorted_ids, const int32_t* offsets,
                                       const float* topk_weights, const uint8_t* W2, const uint16_t* S2,
                                       const uint8_t* Z2, uint16_t* Y, int64_t pairs, int64_t experts, int64_t I,
                                       int64_t H, int64_t group, hipStream_t stream);

extern "C" tb_status tb_fused_moe_w4a16(const uint16_t* X, const float* logits, const uint8_t* W13,
                                        const uint16_t* S13, const uint8_t* Z13, const uint8_t* W2,
                                        const uint16_t* S2, const uint8_t* Z2, uint16_t* out, int64_t tokens,
                                        int64_t experts, int64_t topk, int64_t H, int64_t I, int64_t group13,
                                        int64_t group2, void* workspace, int64_t workspace_bytes,
                                        hipStream_t stream) {
  using namespace tb::moe;
  TB_CHECK_ARG(X && logits && W13 && S13 && Z13 && W2 && S2 && Z2 && out, "tb_fused_moe_w4a16: null pointer");
  TB_CHECK_ARG(tokens > 0 && experts > 0 && topk > 0 && topk <= experts && H > 0 && I > 0,
               "tb_fused_moe_w4a16: need positive sizes and topk <= experts");
  // every step's shape rule, checked before the first launch
  TB_CHECK_ARG(experts <= 1024 && topk <= 32, "tb_fused_moe_w4a16: need experts <= 1024 and topk <= 32");
  TB_CHECK_ARG(tokens * topk < (1ll << 31), "tb_fused_moe_w4a16: tokens * topk must be < 2^31");
  TB_CHECK_ARG(H % 64 == 0 && I % 64 == 0, "tb_fused_moe_w4a16: H and I must be multiples of 64 (H=%lld I=%lld)",
               (long long)H, (long long)I);
  TB_CHECK_ARG(group13 > 0 && group13 % 64 == 0 && H % group13 == 0 && group2 > 0 && group2 % 64 == 0 &&
                   I % group2 == 0,
               "tb_fused_moe_w4a16: groups must be multiples of 64 dividing H (gate/up) and I (down)");
  int64_t need = 0;
  if (tb_status st = tb_fused_moe_w4a16_workspace_size(tokens, topk, experts, H, I, &need)) return st;
  TB_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
               "tb_fused_moe_w4a16: needs a %lld-byte workspace (got %lld)", (long long)need,
               (long long)workspace_bytes);
  TB_CHECK_ALIGN(workspace, 256, "workspace");
  const Workspace ws = carve(workspace, tokens, topk, experts, H, I);
  const int64_t pairs = tokens * topk;
  // dtype 0: fp32 logits -> fp32 weights
  if (tb_status st = tb_moe_topk_gating(logits, ws.w, ws.ids, tokens, experts, topk, 0, stream)) return st;
  if (tb_status st = tb_moe_align(ws.ids, pairs, experts, ws.sorted, ws.offsets, stream)) return st;
  if (tb_status st = tb_moe_w4a16_gate_up(X, ws.sorted, ws.offsets, W13, S13, Z13, ws.act, tokens, topk, experts, H,
                                          I, group13, stream))
    return st;
  if (tb_status st = tb_moe_w4a16_down(ws.act, ws.sorted, ws.offsets, ws.w, W2, S2, Z2, ws.y, pairs, experts, I, H,
                                       group2, stream))
    return st;
  return tb_moe_combine(ws.y, ws.ids, out, tokens, topk, experts, H, stream);
}
