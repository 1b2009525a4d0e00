/*
 * libtbhip — C ABI of the MI355X (gfx950) kernel backend "hip".
 *
 * Every entry point:
 *   - takes raw device pointers, int64 sizes and the hipStream_t to launch on;
 *   - is asynchronous on that stream, allocates no device memory and frees none
 *     (the caller owns every buffer, including any workspace);
 *   - is safe to capture into a hipGraph (no synchronisation, no host<->device
 *     copies, no hipMemset);
 *   - returns TB_OK or an error code, with a message in tb_last_error() (a
 *     thread-local string).  Shape or alignment errors are detected on the host
 *     before anything is launched.
 *
 * fp16 and bf16 buffers are passed as uint16_t bit patterns, fp8-e4m3 (OCP
 * "e4m3fn") as uint8_t codes.  All matrices are row-major and densely packed
 * unless a parameter says otherwise.
 *
 * Int4 weight format ("N-packed, low nibble first"): a logical K x N matrix of
 * 4-bit codes q in [0, 15] is stored as uint8 [K, N/2]; byte [k, j] holds
 * q[k, 2j] in bits 0-3 and q[k, 2j+1] in bits 4-7.  Group-wise parameters run
 * along K with group size G: scales fp16 [K/G, N], zero-points int4 codes
 * packed the same way as uint8 [K/G, N/2].  The dequantised value is
 * fp16((q - z) * s): q - z is exact, the product is rounded once (RNE).
 *
 * Each declaration names the reference (Tilebench) interface it stands in for.
 * The reference drives backends through the Python function
 *     tilebench.benchmarks.operators.<op>.impl_<backend>.run(*inputs, ...)
 * (tilebench/core/engine.py:347-348); the per-operator Python module
 * tilebench_amd/benchmarks/operators/<op>/impl_hip.py binds these symbols with
 * ctypes and keeps that run() signature.
 */
#ifndef TBHIP_H
#define TBHIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int tb_status;
#define TB_OK 0
#define TB_E_INVALID 1   /* bad shape, size or argument                    */
#define TB_E_ALIGN 2     /* a pointer is not aligned as the kernel requires */
#define TB_E_HIP 3       /* a HIP launch or runtime call failed            */
#define TB_E_WORKSPACE 4 /* workspace missing or too small                 */

/* Library version string, e.g. "tbhip 0.1.0 gfx950". */
const char* tb_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char* tb_last_error(void);

/*
 * Int4 group-wise weight dequantisation.
 *   packed uint8 [K, N/2], scales fp16 [K/G, N], zeros uint8 [K/G, N/2]
 *   -> out fp16 [K, N],  out[k, n] = fp16((q[k,n] - z[k/G, n]) * s[k/G, n]).
 * Requires N even, K % G == 0.  The vectorised path needs N % 8 == 0,
 * G % 8 == 0 and 16-byte aligned pointers; other shapes take a scalar path.
 * Replaces: weight_dequant/impl_triton.py:43 run(X, S, M, N, TILE_SIZE)
 * (the reference's dequantisation operator, float X times a tile scale).
 */
tb_status tb_int4_dequant(const uint8_t* packed, const uint16_t* scales, const uint8_t* zeros,
                          uint16_t* out, int64_t K, int64_t N, int64_t group, hipStream_t stream);

/*
 * MoE router gating: per row of logits [M, E], select the
 * k largest logits (descending; equal logits -> lowest expert index first),
 * then weights = softmax over the k selected logits, computed in fp32.
 *   dtype: 0 = fp32, 1 = fp16, 2 = bf16 (logits and weights share it)
 *   logits [M, E] -> weights [M, k] (dtype), indices int32 [M, k].
 * Requires 1 <= k <= min(E, 32) and E <= 1024.
 * Replaces: moe_topk_gating/impl_triton.py:58 run(logits, M, E, k).
 */
tb_status tb_moe_topk_gating(const void* logits, void* weights, int32_t* indices, int64_t M,
                             int64_t E, int64_t k, int dtype, hipStream_t stream);

/*
 * Per-token fp8-e4m3 activation quantisation (step 1).
 *   A fp16 [M, K] -> Aq e4m3 codes uint8 [M, K], sa fp32 [M]
 *   sa[m] = fp32(max_k |A[m,k]|) / 448 (IEEE division),
 *   Aq[m,k] = e4m3(fp32(A[m,k]) / sa[m]): the quotient rounded to fp32, then
 *   to e4m3 round-to-nearest-even without saturation (|x| > 464 -> NaN code).
 *   A row of zeros gives sa = 0 and NaN codes 0xFF (the x86 0/0 result).
 * Requires K % 8 == 0 and 16-byte aligned A and Aq.
 * Replaces: quantize_global/impl_triton.py:31 run(x) (the reference's
 * quantisation operator; it casts to fp16 without scales).
 */
tb_status tb_fp8_act_quant(const uint16_t* A, uint8_t* Aq, float* sa, int64_t M, int64_t K,
                           hipStream_t stream);

/*
 * W4A16 GEMM: Y = fp16(A @ dequant(W)), fp32 accumulation.
 *   A fp16 [M, K], W int4 [K, N] (packed uint8 [K, N/2]), scales fp16 [K/G, N],
 *   zeros uint8 [K/G, N/2] -> Y fp16 [M, N].  Dequantised values are exactly
 *   those of tb_int4_dequant.
 * Requires N % 8 == 0, K % 64 == 0, G % 64 == 0, K % G == 0; A, scales 16-byte
 * aligned.  M <= 16 runs a split-K decode kernel that needs the workspace
 * reported by tb_w4a16_workspace_size (256-byte aligned; zero-filled once when
 * allocated: the kernel leaves its counters at zero after every call, so one
 * workspace serves consecutive calls on one stream; calls that overlap in time
 * must not share a workspace).  Larger M runs the MFMA prefill kernel and
 * needs no workspace.
 * Replaces: matmul_fp32_fp16_fp8/impl_triton.py:124 run(a, b) (the reference's
 * fp16 GEMM operator), with the weight operand kept int4 in HBM.
 */
tb_status tb_w4a16_gemm(const uint16_t* A, const uint8_t* W, const uint16_t* scales, const uint8_t* zeros,
                        uint16_t* Y, int64_t M, int64_t N, int64_t K, int64_t group, void* workspace,
                        int64_t workspace_bytes, hipStream_t stream);

/* Workspace bytes tb_w4a16_gemm needs for this shape (0 if none). */
tb_status tb_w4a16_workspace_size(int64_t M, int64_t N, int64_t K, int64_t group, int64_t* bytes);

/*
 * Slab-contiguous copy of W for the decode below: Wr (K * N / 2 bytes, 16-byte
 * aligned) holds slab s = columns 64 s .. 64 s + 63 as one contiguous run of
 * K / 32 units of 1 KiB; unit u, lane l, word b (4 bytes at byte
 * ((s * K / 32 + u) * 64 + l) * 16 + 4 b) holds the codes of column
 * 64 s + 16 b + l % 16 at rows 32 u + 8 (l / 16) + i, i = 0..7, code i at bit
 * (i % 2) * 16 + (i / 2) * 4.  Requires K % 32 == 0, N % 64 == 0.  A weight
 * format conversion, run once when the weights are loaded (the slab layout is
 * then the weights' stored form for decode; tilebench_amd.formats.
 * w4a16_to_slabs); no operator call runs it or keeps its result.  No
 * counterpart in the reference, which has no W4A16 operator or weight format.
 */
tb_status tb_w4a16_repack_slabs(const uint8_t* W, uint8_t* Wr, int64_t K, int64_t N, hipStream_t stream);

/*
 * W4A16 GEMM for 1 <= M <= 16 from the slab copy: one block per 64-column slab
 * streams its slab over all of K and reduces across its own wavefronts (no
 * split-K, no workspace).  Same operands and result tolerance as
 * tb_w4a16_gemm's decode (fp32 accumulation of the codes, scale and zero-point
 * applied once per group; results reproducible bit for bit).  Requires
 * N % 64 == 0, G in {64, 128}, K in {1024, 2048, 4096}, K % (16 G) == 0; A
 * and Wr 16-byte aligned.  Replaces, for weights stored in the slab layout,
 * the same reference operator as tb_w4a16_gemm (matmul_fp32_fp16_fp8/
 * impl_triton.py:124 run(a, b)).
 */
tb_status tb_w4a16_gemm_slabs(const uint16_t* A, const uint8_t* Wr, const uint16_t* scales, const uint8_t* zeros,
                              uint16_t* Y, int64_t M, int64_t N, int64_t K, int64_t group, hipStream_t stream);

/*
 * tb_w4a16_gemm without a workspace and without any allocation: for callers
 * that cannot allocate device memory (code under hipGraph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  Same operands, results and requirements as tb_w4a16_gemm; the
 * M <= 16 decode keeps its split-K counters and partials in a file-scope
 * device array of the library, 4 MiB + 16 KiB per GPU, held until the process
 * ends (its address is looked up once per device; the first call on a device
 * also clears the counters with a kernel on `stream`).  A shape whose decode
 * needs more than that (only possible on devices with more than 256 CUs) is
 * refused with TB_E_INVALID.  Every call on one GPU shares that GPU's array:
 * calls that overlap in time on one GPU (several streams, or several host
 * threads) race and must not be issued.  Allocates nothing, frees nothing.
 */
tb_status tb_w4a16_gemm_noalloc(const uint16_t* A, const uint8_t* W, const uint16_t* scales, const uint8_t* zeros,
                                uint16_t* Y, int64_t M, int64_t N, int64_t K, int64_t group, hipStream_t stream);

/*
 * Grouped MoE W4A16 GEMM: rows offsets[e] .. offsets[e+1]
 * of the expert-sorted activations A use expert e's int4 weights.
 *   A fp16 [R, K]; W uint8 [E, K, N/2]; scales fp16 [E, K/G, N];
 *   zeros uint8 [E, K/G, N/2]; offsets int32 [E+1] in device memory,
 *   non-decreasing from 0 to R -> Y fp16 [R, N] (rows outside every segment are
 *   left untouched).  Each expert's product is exactly tb_w4a16_gemm's.
 * Requires N % 8 == 0, K % 64 == 0, G % 64 == 0, K % G == 0, E <= 4096,
 * A < 4 GiB, one expert's W < 2 GiB; A, scales, Y 16-byte aligned.
 * Replaces: no reference operator (the reference has no grouped GEMM); the
 * nearest is matmul_fp32_fp16_fp8/impl_triton.py:124 run(a, b) applied per
 * expert.
 */
tb_status tb_moe_w4a16_grouped_gemm(const uint16_t* A, const uint8_t* W, const uint16_t* scales,
                                    const uint8_t* zeros, const int32_t* offsets, uint16_t* Y, int64_t R,
                                    int64_t experts, int64_t N, int64_t K, int64_t group, hipStream_t stream);

/*
 * MoE layer around the grouped W4A16 GEMM (the pipeline's steps are also
 * exported one by one).  Pairs p = t * topk + j are (token, slot) pairs.
 *
 * tb_moe_align: topk_ids int32 [pairs] -> sorted_ids int32 [n_valid], the
 *   pair ids ordered by expert and, within an expert, by p; offsets int32
 *   [E + 1], offsets[e] = number of pairs with an id < e.  Ids outside [0, E)
 *   are routed nowhere.  pairs < 2^31, E <= 4096.
 *
 * tb_moe_w4a16_gate_up: for sorted row m of expert e (offsets[e] <= m <
 *   offsets[e+1]), token t = sorted_ids[m] / topk:
 *     h = fp16(X[t] @ dequant(W13_e)), W13_e int4 [H, 2I] (gate columns 0..I-1,
 *     up columns I..2I-1; packed uint8 [E, H, I], scales fp16 [E, H/G, 2I],
 *     zeros uint8 [E, H/G, I]),
 *     act[m, c] = fp16(silu(fp32(h[c])) * fp32(h[I + c])), silu(x) = x / (1 + exp(-x)).
 *   Requires I % 8 == 0, H % 64 == 0, G % 64 == 0, H % G == 0.
 *
 * tb_moe_w4a16_down: Y[sorted_ids[m]] = fp16(w[sorted_ids[m]] * (act[m] @
 *   dequant(W2_e))) with fp32 weights w [pairs], W2 int4 [E, I, H] (packed
 *   uint8 [E, I, H/2], scales fp16 [E, I/G, H], zeros uint8 [E, I/G, H/2]).
 *   Rows of pairs routed nowhere are not written.  Requires H % 8 == 0,
 *   I % 64 == 0, G % 64 == 0, I % G == 0.
 *
 * tb_moe_combine: out[t] = fp16(sum over slots j in order, skipping ids
 *   outside [0, E), of fp32(Y[t * topk + j])), out fp16 [tokens, H].
 *
 * tb_fused_moe_w4a16: the five steps on one stream: tb_moe_topk_gating of
 *   fp32 router logits [tokens, E] (top-k, softmax over the k values), align,
 *   gate_up, down, combine.  The caller's workspace (size from
 *   tb_fused_moe_w4a16_workspace_size, 256-byte aligned, no clearing needed)
 *   holds weights, ids, the sorted rows, act [pairs, I] and Y [pairs, H].
 *   Requires E <= 1024, topk <= 32, H % 64 == 0, I % 64 == 0, group13 | H,
 *   group2 | I, both groups multiples of 64.
 * Replaces: no reference operator.  The steps follow the reference's
 *   moe_topk_gating (moe_topk_gating/impl_torch.py:4-20) and the config-4
 *   grouped GEMM; the layer itself is the MoE feed-forward block around them.
 */
tb_status tb_moe_align(const int32_t* topk_ids, int64_t pairs, int64_t experts, int32_t* sorted_ids,
                       int32_t* offsets, hipStream_t stream);
tb_status tb_moe_w4a16_gate_up(const uint16_t* X, const int32_t* sorted_ids, const int32_t* offsets,
                               const uint8_t* W13, const uint16_t* S13, const uint8_t* Z13, uint16_t* act,
                               int64_t tokens, int64_t topk, int64_t experts, int64_t H, int64_t I, int64_t group,
                               hipStream_t stream);
tb_status tb_moe_w4a16_down(const uint16_t* act, const int32_t* sorted_ids, const int32_t* offsets,
                            const float* topk_weights, const uint8_t* W2, const uint16_t* S2, const uint8_t* Z2,
                            uint16_t* Y, int64_t pairs, int64_t experts, int64_t I, int64_t H, int64_t group,
                            hipStream_t stream);
tb_status tb_moe_combine(const uint16_t* y, const int32_t* topk_ids, uint16_t* out, int64_t tokens, int64_t topk,
                         int64_t experts, int64_t H, hipStream_t stream);
tb_status tb_fused_moe_w4a16_workspace_size(int64_t tokens, int64_t topk, int64_t experts, int64_t H, int64_t I,
                                            int64_t* bytes);
tb_status tb_fused_moe_w4a16(const uint16_t* X, const float* logits, const uint8_t* W13, const uint16_t* S13,
                             const uint8_t* Z13, const uint8_t* W2, const uint16_t* S2, const uint8_t* Z2,
                             uint16_t* out, int64_t tokens, int64_t experts, int64_t topk, int64_t H, int64_t I,
                             int64_t group13, int64_t group2, void* workspace, int64_t workspace_bytes,
                             hipStream_t stream);

/*
 * Row/column-scaled fp8 GEMM (step 2):
 *   Y bf16 [M, N] = bf16(sa[m] * sw[n] * sum_k e4m3(Aq[m,k]) * e4m3(Wq[k,n])),
 *   fp32 accumulation on the e4m3 matrix cores, one RNE rounding.
 *   Aq uint8 [M, K] row-major; WqT uint8 [N, K] row-major (the K-contiguous
 *   "column-major" weight layout); sa fp32 [M]; sw fp32 [N].
 * Requires K % 128 == 0, N % 8 == 0, each operand < 2 GiB, Aq / WqT / Y
 * 16-byte aligned.
 * Replaces: matmul_fp32_fp16_fp8/impl_triton.py:124 run(a, b) for fp8_e4m3fn
 * (torch._scaled_mm with unit scales and bf16 output in impl_torch.py:21-26),
 * with per-row / per-column scales.
 */
tb_status tb_fp8_scaled_gemm(const uint8_t* Aq, const uint8_t* WqT, const float* sa, const float* sw, uint16_t* Y,
                             int64_t M, int64_t N, int64_t K, hipStream_t stream);

/*
 * Block-scaled fp8 (the 128 x 128 weight-scale blocks of DeepSeek-V3-style
 * fp8 checkpoints, "weight_scale_inv" [ceil(N/128), K/128]):
 *
 * tb_fp8_act_quant_blocks: per token and per block of 128 input channels,
 *   sa[kb, m] = fp32(max_{k in block kb} |A[m,k]|) / 448 and
 *   Aq[m, k] = e4m3(RN32(fp32(A[m,k]) / sa[k/128, m])), the arithmetic of
 *   tb_fp8_act_quant on each block.  A fp16 [M, K]; Aq uint8 [M, K]; sa fp32
 *   [K/128, M] (block-major, M contiguous).  Requires K % 128 == 0, A 16-byte
 *   and Aq 8-byte aligned.
 * tb_fp8_block_gemm: Y bf16 [M, N] =
 *   bf16( sum_kb (sa[kb, m] * sw[n/128, kb]) * sum_{k in block kb} Aq[m,k] * WqT[n,k] ),
 *   the block sums in fp32 on the e4m3 matrix cores, scaled and added in fp32
 *   in block order, one RNE rounding.  WqT uint8 [N, K]; sw fp32
 *   [ceil(N/128), K/128] row-major.  Requires K % 128 == 0, K <= 65536,
 *   N % 8 == 0, each operand < 2 GiB, Aq, WqT and Y 16-byte aligned.
 * Replace: the reference's block-scaled weight dequantisation
 *   (weight_dequant/impl_torch.py:4-8, X * S[i//T, j//T] with T = 128) fused
 *   into its fp8 GEMM (matmul_fp32_fp16_fp8/impl_triton.py:124 run(a, b)).
 */
tb_status tb_fp8_act_quant_blocks(const uint16_t* A, uint8_t* Aq, float* sa, int64_t M, int64_t K,
                                  hipStream_t stream);
tb_status tb_fp8_block_gemm(const uint8_t* Aq, const uint8_t* WqT, const float* sa, const float* sw, uint16_t* Y,
                            int64_t M, int64_t N, int64_t K, hipStream_t stream);

/*
 * The reference's own elementwise dequantisation / quantisation operators.
 * Each product is formed in fp32 and rounded once to the output type (RNE), in
 * the PyTorch reference's order of operations (bit-identical results).
 *
 * tb_weight_dequant: Y[i,j] = X[i,j] * S[i/T, j/T]; X, Y [M, N], S [ceil(M/T),
 *   ceil(N/T)], all of `dtype` (0 fp32, 1 fp16, 2 bf16).
 *   Replaces: weight_dequant/impl_triton.py:43 run(X, S, M, N, TILE_SIZE).
 * tb_dequantize_rowwise: y fp16 [rows, cols] = fp16((state[r] * x[r,c]) * (1/127)),
 *   x int8, state fp32 [rows].
 *   Replaces: dequantize_rowwise/impl_triton.py:43 run(x, state_x).
 * tb_quantize_global: y fp16 [n] = fp16(x fp32 [n]).
 *   Replaces: quantize_global/impl_triton.py:31 run(x).
 */
tb_status tb_weight_dequant(const void* X, const void* S, void* Y, int64_t M, int64_t N, int64_t tile, int dtype,
                            hipStream_t stream);
tb_status tb_dequantize_rowwise(const int8_t* x, const float* state, uint16_t* y, int64_t rows, int64_t cols,
                                hipStream_t stream);
tb_status tb_quantize_global(const float* x, uint16_t* y, int64_t n, hipStream_t stream);

/*
 * The reference's plain GEMM operators (MFMA "NT" GEMM; the second operand is
 * first transposed, unpacked or split into the caller's workspace).
 *
 * tb_matmul_int8: out int32 [M, N] = a int8 [M, K] @ B, where b uint8 [K/4, N]
 *   holds four 2-bit fields per byte and row i*K/4 + kb of B is
 *   ((b[kb, :] >> 2i) & 3) - 1.  Exact integer arithmetic.  Needs K % 128 == 0,
 *   N % 8 == 0 and a workspace of tb_matmul_workspace_size(3, ...) bytes (the
 *   unpacked operand, plus int32 partial planes when the GEMM splits K: grids
 *   of fewer than 256 tiles of 256 x 256 with K >= 2048; every byte it reads
 *   is written by the same call, so it needs no clearing).
 *   Replaces: matmul_int8/impl_triton.py:118 run(a, b) (semantics impl_torch.py:4-19).
 * tb_matmul: dtype 0 fp32, 1 fp16, 2 fp8-e4m3; a [M, K], b [K, N] and out
 *   [M, N] of that dtype.  fp16: fp16(a @ b) with fp32 accumulation.  fp8:
 *   e4m3(bf16(a @ b)) (the reference's unit-scale _scaled_mm to bf16, then its
 *   cast back to e4m3, RNE, no saturation).  fp32: fp32 accumulation of three
 *   bf16 products per term (hi*hi + hi*lo + lo*hi, about 2^-16 relative per
 *   product).  Needs K a multiple of 128 bytes of the dtype (fp32: of 64),
 *   N % 8 == 0 and a workspace of tb_matmul_workspace_size(dtype, ...) bytes.
 *   Replaces: matmul_fp32_fp16_fp8/impl_triton.py:124 run(a, b) (semantics impl_torch.py:21-27).
 * tb_matmul_fp8_bt: the fp8 case with b already transposed to bT [N, K] (the
 *   column-major copy impl_torch.py:10-18 caches per operand pair), no workspace.
 * tb_matmul_workspace_size: workspace bytes for tb_matmul (dtype 0-2) or
 *   tb_matmul_int8 (dtype 3).
 */
tb_status tb_matmul_int8(const int8_t* a, const uint8_t* b, int32_t* out, int64_t M, int64_t N, int64_t K,
                         void* workspace, int64_t workspace_bytes, hipStream_t stream);
tb_status tb_matmul(int dtype, const void* a, const void* b, void* out, int64_t M, int64_t N, int64_t K,
                    void* workspace, int64_t workspace_bytes, hipStream_t stream);
tb_status tb_matmul_fp8_bt(const uint8_t* a, const uint8_t* bT, uint8_t* out, int64_t M, int64_t N, int64_t K,
                           hipStream_t stream);
tb_status tb_matmul_workspace_size(int dtype, int64_t M, int64_t N, int64_t K, int64_t* bytes);

/*
 * Fill `bytes` bytes of `buf` with a 32-bit pattern using a plain store
 * kernel (cache-allocating stores: nontemporal ones would leave the MALL's
 * contents in place).  Used to evict the L2 and the 256 MiB MALL between
 * timed launches (a kernel, not hipMemset, so it may be captured into a graph).
 * Requires bytes % 16 == 0 and a 16-byte aligned buffer.
 * Replaces: tilebench/core/timer.py:107 _flush_l2_cache().
 */
tb_status tb_l2_flush(void* buf, int64_t bytes, uint32_t pattern, hipStream_t stream);

/*
 * Calibration probe: streaming copy dst <- src of `bytes` bytes (16-byte
 * granules, grid-stride), the kernel the measured HBM peak is taken from.
 * Replaces: tilebench/llm/v2/calibration/gpu_probes.py:284 probe_stream().
 */
tb_status tb_probe_copy(const void* src, void* dst, int64_t bytes, hipStream_t stream);

/*
 * Eviction-sweep probe: a streaming read of `bytes` bytes of src (16-byte
 * granules, plain cache-allocating loads).  sink[0] is written only if the
 * XOR of a granule's four words equals `key` (pick a key the data cannot
 * produce, so nothing is written).  The re-read probe placed behind flushes of
 * growing size to find the last-level cache's eviction size.
 * Replaces: the re-read probe of the reference's eviction sweep, described at
 * tilebench/hardware.py:24-37.
 */
tb_status tb_probe_read(const void* src, int64_t bytes, uint32_t key, uint32_t* sink, hipStream_t stream);

/*
 * Calibration probe: `blocks` x 256 threads, each wavefront issuing
 * 8 * iters independent MFMAs (kind 0: v_mfma_f32_32x32x16_f16, 32768 flop
 * each; kind 1: v_mfma_f32_32x32x64_f8f6f4 on e4m3, 131072 flop each; kind 2:
 * v_mfma_f32_32x32x16_bf16, 32768 flop each; kind 3: v_mfma_i32_32x32x32_i8,
 * 65536 op each), then one float per thread into out[blocks * 256].  The
 * instruction-level MFMA ceiling of the calibration is taken from it.
 * Replaces: tilebench/llm/v2/calibration/gpu_probes.py:225 probe_gemm().
 */
tb_status tb_probe_mfma(int kind, int64_t blocks, int64_t iters, float* out, hipStream_t stream);

/*
 * Clock probe: `blocks` x 256 threads running the fp16 loop of tb_probe_mfma
 * (kind 0) between two reads of the shader clock counter and of the constant
 * 100 MHz counter; block b writes the two differences to clocks[2b] and
 * clocks[2b + 1] (its average shader clock is 100 MHz x their ratio) and one
 * float per wavefront to sink[4 * blocks].  Shows how the clock under an
 * MFMA-bound load depends on what ran before (tilebench_amd.profiling.clock).
 * No counterpart in the reference: a probe of this backend's measurement
 * conditions, beside the calibration probes above.
 */
tb_status tb_probe_clock(int64_t blocks, int64_t iters, uint64_t* clocks, float* sink, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TBHIP_H */
