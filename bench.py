"""Benchmark of the hip backend's hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--op NAME] [--no-cpu-baseline]
    (defaults: K = 100, W = 20)

A step is one launch of the operator on one batch of seeded synthetic input
already resident in HBM.  W untimed warmup steps, then exactly K steps captured
into one hipGraph and replayed between two hipEvents on the stream the kernels
run on (bracketed by torch.cuda.synchronize()).  Steps rotate over copies of
the input at distinct addresses, together larger than 2x the 256 MiB MALL, so
no step finds its operands in the last-level cache.  Prints ONE JSON line with the driver's fields plus:

  roofline      achieved GB/s or TFLOP/s of the operator's kernel (algorithmic
                bytes or flops per launch / mean launch time from the events),
                MI355X's published peak and the fraction, and the peak this
                GPU reaches in the same process (measured_peak: the copy or
                MFMA probe of the library) with the fraction of it;
  cpu_baseline  the numpy CPU oracle timed on the host cores on a bounded slice
                of the same workload (the oracle is used only as this timed CPU
                port, never on the GPU path);
  suite         (--suite) the same measurement for every BASELINE config.

The default workload is BASELINE config 1 at M = 4096 (the W4A16 GEMM the
metric quotes in TFLOP/s).  Only one GPU is used: --gpus above 1 exits.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# MI355X published peaks (dense): HBM3E 8 TB/s; MFMA fp16/bf16 2.5 PFLOP/s, fp8 5.0 PFLOP/s,
# int8 5.0 POP/s, fp32 157.3 TFLOP/s.
PEAK_HBM_GBS = 8000.0
PEAK_TFLOPS = {"fp16": 2500.0, "bf16": 2500.0, "fp8": 5000.0, "int8": 5000.0, "fp32": 157.3}


# ----------------------------------------------------------------------------- workloads
# Each workload: inputs(), step(inputs) (the hip kernel launch, async), the
# algorithmic work per launch, the roofline it is bound by, and a CPU sample.

def _w_int4_dequant():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.int4_dequant import impl_hip

    K, N, G = 4096, 4096, 128
    nbytes = K * N // 2 + (K // G) * N * 2 + (K // G) * N // 2 + K * N * 2

    def inputs():
        return T.generate_int4_dequant_inputs(K, N, G, seed=0, device="cuda")

    def cpu_sample():
        import oracle
        p, s, z, *_ = T.generate_int4_dequant_inputs(K, N, G, seed=0, device="cpu")
        p, s, z = p.numpy(), s.numpy(), z.numpy()
        return (lambda: oracle.int4_dequant(p, s, z, G)), nbytes, "full config 0 (K=N=4096), numpy"

    return dict(name="int4_dequant", config={"workload": "int4_dequant", "K": K, "N": N, "group": G},
                metric="int4 dequant HBM throughput", unit="GB/s", dtype="int4->fp16", bound="hbm",
                bytes=nbytes, flops=2 * K * N, inputs=inputs, step=lambda x: impl_hip.run(*x),
                kernel="tb::int4_dequant_vec<8>", cpu_sample=cpu_sample)


def _w_gating(E):
    def make():
        from tilebench_amd.data import tensors as T
        from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_hip

        M, k = 16384, 8
        nbytes = M * E * 4 + M * k * 4 + M * k * 4

        def inputs():
            return T.generate_moe_topk_gating_inputs(M, E, k, seed=3, device="cuda")

        def cpu_sample():
            import oracle
            lg = T.generate_moe_topk_gating_inputs(M, E, k, seed=3, device="cpu")[0].numpy()
            return (lambda: oracle.moe_topk_gating(lg, k)), nbytes, f"full config 3 (M=16384, E={E}), numpy"

        return dict(name=f"moe_topk_gating_E{E}", config={"workload": "moe_topk_gating", "M": M, "E": E, "k": k},
                    metric="MoE gating HBM throughput", unit="GB/s", dtype="fp32", bound="hbm", bytes=nbytes,
                    flops=None, inputs=inputs, step=lambda x: impl_hip.run(*x), kernel=f"tb::filter_kernel<0, {E // 16}, 8>",
                    cpu_sample=cpu_sample)
    return make


def _w_gating_reference_grid():
    import torch
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_hip

    M, E, k = 20480, 128, 2
    nbytes = M * E * 2 + M * k * 2 + M * k * 4       # moe_topk_gating/config.yaml bytes_expr, fp16

    def inputs():
        return T.generate_moe_topk_gating_inputs(M, E, k, dtype=torch.float16, dist="grid", seed=3, device="cuda")

    def cpu_sample():
        import oracle
        lg = T.generate_moe_topk_gating_inputs(M, E, k, dtype=torch.float16, dist="grid", seed=3,
                                               device="cpu")[0].numpy()
        return (lambda: oracle.moe_topk_gating(lg, k, dtype="fp16")), nbytes, "full M=20480, E=128, k=2, fp16, numpy"

    return dict(name="moe_topk_gating_ref_grid",
                config={"workload": "moe_topk_gating", "M": M, "E": E, "k": k, "dtype": "fp16", "dist": "grid"},
                metric="MoE gating HBM throughput", unit="GB/s", dtype="fp16", bound="hbm", bytes=nbytes,
                flops=None, inputs=inputs, step=lambda x: impl_hip.run(*x), kernel="tb::gating_kernel<1, 16, 8, 2>",
                cpu_sample=cpu_sample)


def _w_fp8_quant():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.fp8_act_quant import impl_hip

    M = K = 8192
    nbytes = 2 * M * K + M * K + 4 * M

    def inputs():
        return T.generate_fp8_act_quant_inputs(M, K, seed=2, device="cuda")

    def cpu_sample():
        import oracle
        rows = 1024
        A = T.generate_fp8_act_quant_inputs(rows, K, seed=2, device="cpu")[0].numpy()
        return (lambda: oracle.fp8_act_quant(A)), 3 * rows * K + 4 * rows, f"{rows} of 8192 rows, numpy"

    return dict(name="fp8_act_quant", config={"workload": "fp8_act_quant", "M": M, "K": K},
                metric="fp8 per-token quant HBM throughput", unit="GB/s", dtype="fp16->e4m3", bound="hbm",
                bytes=nbytes, flops=None, inputs=inputs, step=lambda x: impl_hip.run(*x), kernel="tb::fp8_quant_rows<4>",
                cpu_sample=cpu_sample)


def _w_w4a16(M):
    def make():
        from tilebench_amd.data import tensors as T
        from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip

        K, N, G = 4096, 11008, 128
        flops = 2 * M * K * N
        nbytes = 2 * M * K + K * N // 2 + (K // G) * N * 2 + (K // G) * N // 2 + 2 * M * N

        def inputs():
            return T.generate_w4a16_gemm_inputs(M, K, N, G, seed=1, device="cuda")

        def cpu_sample():
            import oracle
            rows = min(M, 64)
            A, p, s, z, _ = T.generate_w4a16_gemm_inputs(rows, K, N, G, seed=1, device="cpu")
            A, p, s, z = A.numpy(), p.numpy(), s.numpy(), z.numpy()
            work = 2 * rows * K * N if M > 16 else nbytes
            return ((lambda: oracle.w4a16_gemm(A, p, s, z, G)), work,
                    f"{rows} of {M} rows (numpy int4 dequant + fp32 BLAS matmul)")

        big = M > 16
        return dict(name=f"w4a16_gemm_M{M}",
                    config={"workload": "w4a16_gemm", "M": M, "K": K, "N": N, "group": G},
                    metric="W4A16 GEMM throughput" if big else "W4A16 decode GEMM HBM throughput",
                    unit="TFLOP/s" if big else "GB/s", dtype="fp16 x int4 -> fp16 (fp32 acc)",
                    bound="mfma" if big else "hbm", peak_key="fp16", bytes=nbytes, flops=flops, out_bytes=2 * M * N,
                    inputs=inputs, step=lambda x: impl_hip.run(*x),
                    kernel="tb::w4a16::w4a16_prefill" if big else "tb::w4a16::w4a16_decode<false>", cpu_sample=cpu_sample)
    return make


def _w_fp8_gemm():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.fp8_scaled_gemm import impl_hip

    M = N = K = 8192
    flops = 2 * M * N * K
    nbytes = M * K + K * N + 4 * M + 4 * N + 2 * M * N

    def inputs():
        return T.generate_fp8_scaled_gemm_inputs(M, N, K, seed=2, device="cuda")

    def cpu_sample():
        import oracle
        import torch
        rows = 32
        Aq, Wq, sa, sw = T.generate_fp8_scaled_gemm_inputs(rows, N, K, seed=2, device="cpu")
        a, w = Aq.view(torch.uint8).numpy(), Wq.contiguous().view(torch.uint8).numpy()
        sa, sw = sa.numpy(), sw.numpy()
        return ((lambda: oracle.fp8_scaled_gemm(a, w, sa, sw)), 2 * rows * N * K,
                f"{rows} of {M} rows (numpy e4m3 decode + float64 BLAS matmul)")

    return dict(name="fp8_scaled_gemm", config={"workload": "fp8_scaled_gemm", "M": M, "N": N, "K": K},
                metric="fp8 row/column-scaled GEMM throughput", unit="TFLOP/s", dtype="e4m3 x e4m3 -> bf16 (fp32 acc)",
                bound="mfma", peak_key="fp8", bytes=nbytes, flops=flops, out_bytes=2 * M * N, inputs=inputs,
                step=lambda x: impl_hip.run(*x), kernel="tb::fp8gemm::fp8_gemm_kernel", cpu_sample=cpu_sample)


def _w_grouped():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.moe_w4a16_grouped_gemm import impl_hip

    tokens, topk, E, K, N, G = 16384, 8, 64, 4096, 1408, 128
    flops = 2 * tokens * topk * K * N
    nbytes = 2 * tokens * topk * K + E * (K * N // 2 + (K // G) * N * 2 + (K // G) * N // 2) + 2 * tokens * topk * N

    def inputs():
        return T.generate_moe_w4a16_grouped_gemm_inputs(tokens, topk, E, K, N, G, seed=4, device="cuda")

    def cpu_sample():
        import oracle
        A, p, s, z, off, _ = T.generate_moe_w4a16_grouped_gemm_inputs(256, 8, E, K, N, G, seed=4, device="cpu")
        A, p, s, z, off = A.numpy(), p.numpy(), s.numpy(), z.numpy(), off.numpy()
        return ((lambda: oracle.moe_w4a16_grouped_gemm(A, p, s, z, off, G)), 2 * 256 * 8 * K * N,
                "256 of 16384 tokens x top-8 over all 64 experts (numpy dequant + fp32 BLAS)")

    return dict(name="moe_w4a16_grouped_gemm",
                config={"workload": "moe_w4a16_grouped_gemm", "tokens": tokens, "topk": topk, "experts": E, "K": K,
                        "N": N, "group": G, "zipf_s": 1.1, "pad": 128},
                metric="MoE grouped W4A16 GEMM throughput", unit="TFLOP/s", dtype="fp16 x int4 -> fp16 (fp32 acc)",
                bound="mfma", peak_key="fp16", bytes=nbytes, flops=flops, out_bytes=2 * (tokens * topk + E * 128) * N,
                inputs=inputs, step=lambda x: impl_hip.run(*x), kernel="tb::w4a16::w4a16_grouped", cpu_sample=cpu_sample)


def _w_fused_moe():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.fused_moe_w4a16 import impl_hip

    tokens, E, topk, H, I, G13, G2 = 16384, 64, 8, 4096, 704, 128, 64
    flops = 6 * tokens * topk * H * I           # gate/up 2*T*k*H*2I + down 2*T*k*I*H
    wbytes = E * (H * I + (H // G13) * 2 * I * 2 + (H // G13) * I + I * H // 2 + (I // G2) * H * 2 + (I // G2) * H // 2)
    nbytes = 2 * tokens * H + 4 * tokens * E + wbytes + 2 * tokens * H

    def inputs():
        return T.generate_fused_moe_w4a16_inputs(tokens, E, topk, H, I, G13, G2, seed=15, device="cuda")

    def cpu_sample():
        import oracle
        x = T.generate_fused_moe_w4a16_inputs(256, E, topk, H, I, G13, G2, seed=15, device="cpu")
        x = [t.numpy() if hasattr(t, "numpy") else t for t in x]
        return ((lambda: oracle.fused_moe_w4a16(*x)), 6 * 256 * topk * H * I,
                "256 of 16384 tokens through the whole layer, all 64 experts (numpy dequant + fp32 BLAS)")

    return dict(name="fused_moe_w4a16",
                config={"workload": "fused_moe_w4a16", "tokens": tokens, "experts": E, "topk": topk, "H": H, "I": I,
                        "group13": G13, "group2": G2, "zipf_s": 1.1},
                metric="MoE layer (gating + sort + W4A16 gate/up + SiLU + W4A16 down + combine) throughput",
                unit="TFLOP/s", dtype="fp16 x int4 -> fp16 (fp32 acc)", bound="mfma", peak_key="fp16",
                bytes=nbytes, flops=flops, out_bytes=2 * tokens * H, inputs=inputs, step=lambda x: impl_hip.run(*x),
                kernel="tb::w4a16::moe_gate_up", cpu_sample=cpu_sample)


def _w_weight_dequant():
    import torch
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.weight_dequant import impl_hip

    M, TS = 10240, 128
    nbytes = 2 * M * M * 2 + ((M + TS - 1) // TS) ** 2 * 2   # weight_dequant/config.yaml bytes_expr, fp16

    def inputs():
        return T.generate_weight_dequant_inputs(M, TS, dtype=torch.float16, seed=10, device="cuda")

    def cpu_sample():
        import oracle
        rows = 1024
        X, S, *_ = T.generate_weight_dequant_inputs(rows, TS, dtype=torch.float16, N=M, seed=10, device="cpu")
        X, S = X.numpy(), S.numpy()
        return (lambda: oracle.weight_dequant(X, S, TS, "fp16")), 4 * rows * M, f"{rows} of {M} rows, fp16, numpy"

    return dict(name="weight_dequant", config={"workload": "weight_dequant", "M": M, "TILE_SIZE": TS, "dtype": "fp16"},
                metric="weight_dequant HBM throughput", unit="GB/s", dtype="fp16", bound="hbm", bytes=nbytes,
                flops=M * M, inputs=inputs, step=lambda x: impl_hip.run(*x), kernel="tb::analog::weight_dequant_vec<1>",
                cpu_sample=cpu_sample)


def _w_dequantize_rowwise():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.dequantize_rowwise import impl_hip

    rows, cols = 4096, 8192
    nbytes = rows * cols + rows * 4 + rows * cols * 2            # dequantize_rowwise/config.yaml bytes_expr

    def inputs():
        return T.generate_dequantize_rowwise_inputs(rows, cols, seed=11, device="cuda")

    def cpu_sample():
        import oracle
        x, st = T.generate_dequantize_rowwise_inputs(rows, cols, seed=11, device="cpu")
        x, st = x.numpy(), st.numpy()
        return (lambda: oracle.dequantize_rowwise(x, st)), nbytes, "full 4096x8192, numpy"

    return dict(name="dequantize_rowwise", config={"workload": "dequantize_rowwise", "rows": rows, "cols": cols},
                metric="dequantize_rowwise HBM throughput", unit="GB/s", dtype="int8->fp16", bound="hbm",
                bytes=nbytes, flops=2 * rows * cols, inputs=inputs, step=lambda x: impl_hip.run(*x),
                kernel="tb::analog::dequant_rowwise_rows", cpu_sample=cpu_sample)


def _w_quantize_global():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.quantize_global import impl_hip

    n = 20 * 1024 * 1024
    nbytes = n * 4 + n * 2

    def inputs():
        return T.generate_quantize_global_inputs(n, seed=12, device="cuda")

    def cpu_sample():
        import oracle
        x = T.generate_quantize_global_inputs(n, seed=12, device="cpu")[0].numpy()
        return (lambda: oracle.quantize_global(x)), nbytes, "full n=20Mi, numpy"

    return dict(name="quantize_global", config={"workload": "quantize_global", "n": n},
                metric="quantize_global HBM throughput", unit="GB/s", dtype="fp32->fp16", bound="hbm", bytes=nbytes,
                flops=None, inputs=inputs, step=lambda x: impl_hip.run(*x), kernel="tb::analog::f32_to_f16_vec",
                cpu_sample=cpu_sample)


def _w_matmul_int8():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.matmul_int8 import impl_hip

    M = N = 2048
    K = 20480
    nbytes = M * K + K * N // 4 + 4 * M * N          # matmul_int8/config.yaml bytes_expr

    def inputs():
        return T.generate_matmul_int8_inputs(M, N, K, seed=13, device="cuda")

    def cpu_sample():
        import oracle
        rows = 256
        a, b = T.generate_matmul_int8_inputs(M, N, K, seed=13, device="cpu")
        a, b = a.numpy()[:rows], b.numpy()
        return (lambda: oracle.matmul_int8(a, b)), 2 * rows * N * K, f"{rows} of {M} rows, numpy float64 BLAS (exact)"

    return dict(name="matmul_int8", config={"workload": "matmul_int8", "M": M, "N": N, "K": K},
                metric="matmul_int8 throughput", unit="TFLOP/s", dtype="int8 x int2 -> int32", bound="mfma",
                peak_key="int8", bytes=nbytes, flops=2 * M * N * K, inputs=inputs, step=lambda x: impl_hip.run(*x),
                kernel="tb::ntg::nt_gemm<3, 4, 256, 256, 128, 64>", cpu_sample=cpu_sample)


def _w_matmul(dt):
    def make():
        import torch
        from tilebench_amd.data import tensors as T
        from tilebench_amd.benchmarks.operators.matmul_fp32_fp16_fp8 import impl_hip

        M = N = 4096
        K = 20480
        tdt = {"fp32": torch.float32, "fp16": torch.float16, "fp8_e4m3fn": torch.float8_e4m3fn}[dt]
        esz = {"fp32": 4, "fp16": 2, "fp8_e4m3fn": 1}[dt]
        nbytes = (M * K + K * N + M * N) * esz          # matmul_fp32_fp16_fp8/config.yaml bytes_expr

        def inputs():
            return T.generate_matmul_fp32_fp16_fp8_inputs(M, N, K, dtype=tdt, seed=14, device="cuda")

        def cpu_sample():
            import oracle
            rows = 64
            a, b = T.generate_matmul_fp32_fp16_fp8_inputs(M, N, K, dtype=tdt, seed=14, device="cpu")
            if dt == "fp8_e4m3fn":
                a8, b8 = a.view(torch.uint8).numpy()[:rows], b.view(torch.uint8).numpy()
                fn = lambda: oracle.matmul_fp8(a8, b8)
            elif dt == "fp16":
                a16, b16 = a.numpy()[:rows], b.numpy()
                fn = lambda: oracle.matmul_f16(a16, b16)
            else:
                a32, b32 = a.numpy()[:rows], b.numpy()
                fn = lambda: oracle.matmul_f32(a32, b32)
            return fn, 2 * rows * N * K, f"{rows} of {M} rows, numpy float64 BLAS"

        kern = {"fp32": "tb::ntg::nt_gemm<2, 3, 256, 256, 128, 64>", "fp16": "tb::ntg::nt_gemm<1, 2, 256, 256, 128, 64>",
                "fp8_e4m3fn": "tb::ntg::nt_gemm<0, 1, 256, 256, 128, 64>"}[dt]
        peak = {"fp32": "fp32", "fp16": "fp16", "fp8_e4m3fn": "fp8"}[dt]
        return dict(name=f"matmul_{dt}", config={"workload": "matmul_fp32_fp16_fp8", "M": M, "N": N, "K": K, "dtype": dt},
                    metric="matmul throughput", unit="TFLOP/s", dtype=dt if dt != "fp32" else "fp32 (3 x bf16 products)",
                    bound="mfma", peak_key=peak, bytes=nbytes, flops=2 * M * N * K, inputs=inputs,
                    step=lambda x: impl_hip.run(*x), kernel=kern, cpu_sample=cpu_sample)
    return make


def _w_copy():
    import torch

    nbytes = 1 << 30

    def inputs():
        return (torch.empty(nbytes // 2, dtype=torch.uint8, device="cuda"),)

    def step(x):
        from tilebench_amd import runtime as rt
        src = x[0]
        dst = torch.empty_like(src)
        rt.call("tb_probe_copy", src.data_ptr(), dst.data_ptr(), src.numel(), rt.stream_handle())
        return dst

    return dict(name="hbm_copy_probe", config={"workload": "hbm_copy_probe", "bytes": nbytes},
                metric="HBM streaming copy (calibration probe)", unit="GB/s", dtype="u8", bound="hbm", bytes=nbytes,
                flops=None, out_bytes=nbytes // 2, inputs=inputs, step=step, kernel="tb::copy_kernel", cpu_sample=None)


WORKLOADS = {
    "w4a16_gemm_M4096": _w_w4a16(4096),
    "w4a16_gemm_M16": _w_w4a16(16),
    "w4a16_gemm_M1": _w_w4a16(1),
    "int4_dequant": _w_int4_dequant,
    "moe_topk_gating_E64": _w_gating(64),
    "moe_topk_gating_E256": _w_gating(256),
    "moe_topk_gating_ref_grid": _w_gating_reference_grid,
    "fp8_act_quant": _w_fp8_quant,
    "fp8_scaled_gemm": _w_fp8_gemm,
    "moe_w4a16_grouped_gemm": _w_grouped,
    "fused_moe_w4a16": _w_fused_moe,
    "weight_dequant": _w_weight_dequant,
    "dequantize_rowwise": _w_dequantize_rowwise,
    "quantize_global": _w_quantize_global,
    "matmul_int8": _w_matmul_int8,
    "matmul_fp16": _w_matmul("fp16"),
    "matmul_fp8": _w_matmul("fp8_e4m3fn"),
    "matmul_fp32": _w_matmul("fp32"),
    "hbm_copy_probe": _w_copy,
}
DEFAULT_OP = "w4a16_gemm_M4096"


# ----------------------------------------------------------------------------- measurement

MALL_BYTES = 256 * 1024 * 1024


def _footprint(x) -> int:
    import torch
    return sum(t.numel() * t.element_size() for t in x if isinstance(t, torch.Tensor))


def input_sets(w, x) -> list:
    """The inputs plus device copies at other addresses, enough that one pass
    over all sets moves more than 2x the 256 MiB MALL: consecutive steps then
    never find their operands in the cache (the reference evicts the LLC
    before every timed launch, tilebench/core/timer.py:81-117)."""
    import torch
    per_set = _footprint(x) + w.get("out_bytes", 0)
    n = max(1, min(64, -(-2 * MALL_BYTES // max(per_set, 1))))
    sets = [x]
    for _ in range(n - 1):
        sets.append(tuple(t.clone() if isinstance(t, torch.Tensor) else t for t in x))
    return sets


def time_steps(w, sets, steps: int, warmup: int):
    """Mean ms per step: `steps` launches captured into one hipGraph (no host
    work between launches), replayed between two hipEvents on the stream the
    kernels are launched on.  Step i uses input set i mod len(sets); outputs
    live in a ring of 8 buffers (fresh allocations, as each reference run()
    makes, without holding `steps` of them).  A replay carries a fixed start-up
    cost of about a millisecond on this GPU, so the default of 100 steps keeps
    it below a few percent of the mean."""
    import torch

    for i in range(max(1, warmup)):
        w["step"](sets[i % len(sets)])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    keep = []
    with torch.cuda.graph(graph):
        for i in range(steps):
            keep.append(w["step"](sets[i % len(sets)]))
            if len(keep) > 8:
                keep.pop(0)
    graph.replay()  # upload + warm the instruction cache
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    graph.replay()
    stop.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    del keep, graph
    return ms


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (profiles/traffic.json), or None if it was not profiled."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            k = json.load(f)["kernels"].get(kernel)
    except (OSError, ValueError, KeyError):
        return None
    return None if k is None else int(k["fetch_bytes"] + k["write_bytes"])


_MEASURED_PEAKS: dict = {}


def measured_peak(bound: str, peak_key: str | None):
    """The peak this GPU reaches now, measured in this process with the
    library's probes: HBM GB/s from tb_probe_copy over 512 MiB each way, matrix
    TFLOP/s from tb_probe_mfma (fp16 32x32x16 or fp8 32x32x64 MFMAs back to back,
    two 4-wavefront blocks per CU).  None for a matrix type the probe does not
    cover (int8, fp32).  Each figure is the mean of 10 back-to-back launches
    after 3 untimed ones, measured once per process."""
    import torch
    from tilebench_amd import runtime as rt

    key = "hbm" if bound == "hbm" else peak_key
    if key in _MEASURED_PEAKS:
        return _MEASURED_PEAKS[key]
    stream = rt.stream_handle()
    if key == "hbm":
        n = 512 * 1024 * 1024
        src = torch.empty(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        launch = lambda: rt.call("tb_probe_copy", src.data_ptr(), dst.data_ptr(), n, stream)  # noqa: E731
        work, scale = 2 * n, 1e9
    elif key in ("fp16", "fp8"):
        kind = 0 if key == "fp16" else 1
        blocks, iters = 2 * torch.cuda.get_device_properties(0).multi_processor_count, 2000
        out = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
        launch = lambda: rt.call("tb_probe_mfma", kind, blocks, iters, out.data_ptr(), stream)  # noqa: E731
        work, scale = blocks * 4 * 8 * iters * (32768 if kind == 0 else 131072), 1e12
    else:
        _MEASURED_PEAKS[key] = None
        return None
    for _ in range(3):
        launch()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        launch()
    e1.record()
    torch.cuda.synchronize()
    _MEASURED_PEAKS[key] = round(work / (e0.elapsed_time(e1) / 10 * 1e-3) / scale, 2)
    return _MEASURED_PEAKS[key]


def roofline(w, ms: float) -> dict:
    if w["bound"] == "hbm":
        achieved = w["bytes"] / (ms * 1e-3) / 1e9
        peak, unit = PEAK_HBM_GBS, "GB/s"
    else:
        achieved = w["flops"] / (ms * 1e-3) / 1e12
        peak, unit = PEAK_TFLOPS[w["peak_key"]], "TFLOP/s"
    mp = measured_peak(w["bound"], w.get("peak_key"))
    return {"bound": w["bound"], "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": measured_traffic(w["kernel"]),
            "kernel": w["kernel"], "measured_peak": mp,
            "frac_of_measured": None if mp is None else round(achieved / mp, 4)}


def cpu_baseline(w, budget_s: float = 10.0) -> dict:
    """Time the CPU oracle on the workload's bounded sample (rank 0, N=1 only)."""
    import torch

    fn, work, sample = w["cpu_sample"]()
    t0 = time.perf_counter()
    fn()  # warmup, also sizes the repeat count
    one = time.perf_counter() - t0
    reps = max(1, min(50, int(budget_s / max(one, 1e-6))))
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    dt = (time.perf_counter() - t0) / reps
    value = work / dt / (1e9 if w["unit"] == "GB/s" else 1e12)
    threads = int(os.environ.get("OMP_NUM_THREADS") or torch.get_num_threads())
    return {"value": round(value, 4), "unit": w["unit"], "cores": threads, "kind": "port",
            "sample": f"{sample}; {reps} reps, {dt * 1e3:.1f} ms each, host has {os.cpu_count()} CPUs"}


def measure(name: str, steps: int, warmup: int, with_cpu: bool) -> dict:
    import torch

    w = WORKLOADS[name]()
    sets = input_sets(w, w["inputs"]())
    torch.cuda.synchronize()
    ms = time_steps(w, sets, steps, warmup)
    out = {"name": w["name"], "w": w, "ms": ms, "roofline": roofline(w, ms), "input_sets": len(sets)}
    if with_cpu and w.get("cpu_sample"):
        out["cpu_baseline"] = cpu_baseline(w)
    del sets
    torch.cuda.empty_cache()
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--op", default=DEFAULT_OP, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--suite", action="store_true", help="also measure every other workload")
    ap.add_argument("--only", default=None, help="comma-separated workloads for --suite (default: all)")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path.",
              file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    from tilebench_amd import runtime as rt

    rt.require_device()
    rt.load_library()

    main_res = measure(args.op, args.steps, args.warmup, not args.no_cpu_baseline)
    w, ms = main_res["w"], main_res["ms"]
    value = main_res["roofline"]["achieved"]
    line = {
        "metric": w["metric"], "value": value, "unit": w["unit"], "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": w["dtype"], "data": "synthetic (seeded CPU generator, resident in HBM)",
        "config": {**w["config"], "input_sets": main_res["input_sets"]}, "roofline": main_res["roofline"],
        "cpu_baseline": main_res.get("cpu_baseline"),
    }
    if args.suite:
        suite = {}
        names = args.only.split(",") if args.only else list(WORKLOADS)
        for name in names:
            if name == args.op:
                continue
            r = measure(name, args.steps, args.warmup, False)
            suite[name] = {"ms": round(r["ms"], 6), **r["roofline"]}
        line["suite"] = suite
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
