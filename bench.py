"""Benchmark of the hip backend's hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--op NAME] [--no-suite] [--suite]
                    [--no-cpu-baseline]
    (defaults: K = 100, W = 20)

A step is one launch of the operator on one batch of seeded synthetic input
already resident in HBM.  W untimed warmup steps run eagerly, then one eager
step on every input copy; then K steps are captured into one hipGraph.  A second graph of the same K steps over other
copies of the inputs is replayed first, untimed (as many times as take at
least WARM_MS = 200 ms and move 2x the MALL), so the GPU is busy and at its
sustained clock when the timed graph starts; the timed graph is replayed between
two hipEvents on the stream the kernels run on, with torch.cuda.synchronize()
before the untimed replay and after the stop event.  The timed steps read
input copies that no launch has touched for at least 2x the 256 MiB MALL of
other traffic, so no timed step finds its operands in the last-level cache.
Prints ONE JSON line with the driver's fields plus:

  roofline      achieved GB/s or TFLOP/s of the operator's kernel (algorithmic
                bytes or flops per launch / mean launch time from the events),
                MI355X's published peak and the fraction, the peak this GPU
                reaches in the same process by the calibration protocol
                (measured_peak, frac_of_measured) and the committed calibration
                of the same protocol (calibrated_peak, frac_of_calibrated);
  cpu_baseline  the PyTorch CPU reference (impl_torch.run of the operator) on
                CPU copies of the same seeded inputs, on a bounded sample of the
                workload, warmup 1 and repeat 3, with every host core torch may
                use (torch.set_num_threads), the core count and the CPU model;
  suite         every other BASELINE config measured the same way (each with
                its own roofline and cpu_baseline); --suite adds the
                reference's analog operators, the MoE layer and the copy probe.

The headline workload is BASELINE config 1 at M = 4096 (the W4A16 GEMM the
metric quotes in TFLOP/s).  Only one GPU is used: --gpus above 1 exits.
"""
from __future__ import annotations

import argparse
import json
import math
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
#: bench peak key -> key of the calibrated peak file (tilebench_amd/calibration.py)
CALIBRATION_KEY = {"fp16": "fp16_mma", "bf16": "bf16_mma", "fp8": "fp8_e4m3fn_mma", "int8": "int8_mma"}

MiB = 1024 * 1024
MALL_BYTES = 256 * MiB
WARM_MS = 200.0  # untimed back-to-back work before every timed replay (clock at its sustained level)


# ----------------------------------------------------------------------------- workloads
# Each workload: inputs() on the GPU, step(inputs) (the hip kernel launch,
# asynchronous), the algorithmic work per launch and the roofline bounding it,
# and cpu() -> (callable, work of one call, sample description): the PyTorch
# reference (impl_torch.run) on CPU tensors of a bounded sample.

def _w_int4_dequant():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.int4_dequant import impl_hip, impl_torch

    K, N, G = 4096, 4096, 128
    nbytes = K * N // 2 + (K // G) * N * 2 + (K // G) * N // 2 + K * N * 2

    def cpu():
        x = T.generate_int4_dequant_inputs(K, N, G, seed=0, device="cpu")
        return (lambda: impl_torch.run(*x)), nbytes, "full config 0 (K = N = 4096)"

    return dict(name="int4_dequant", config={"workload": "int4_dequant", "K": K, "N": N, "group": G},
                metric="int4 dequant HBM throughput", unit="GB/s", dtype="int4->fp16", bound="hbm",
                bytes=nbytes, flops=2 * K * N, out_bytes=K * N * 2,
                inputs=lambda: T.generate_int4_dequant_inputs(K, N, G, seed=0, device="cuda"),
                step=lambda x: impl_hip.run(*x), kernel="tb::int4_dequant_vec<8>", cpu=cpu)


def _w_gating(E):
    def make():
        from tilebench_amd.data import tensors as T
        from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_hip, impl_torch

        M, k = 16384, 8
        nbytes = M * E * 4 + M * k * 4 + M * k * 4

        def cpu():
            x = T.generate_moe_topk_gating_inputs(M, E, k, seed=3, device="cpu")
            return (lambda: impl_torch.run(*x)), nbytes, f"full config 3 (M = 16384, E = {E})"

        return dict(name=f"moe_topk_gating_E{E}", config={"workload": "moe_topk_gating", "M": M, "E": E, "k": k},
                    metric="MoE gating HBM throughput", unit="GB/s", dtype="fp32", bound="hbm", bytes=nbytes,
                    flops=None, out_bytes=M * k * 8,
                    inputs=lambda: T.generate_moe_topk_gating_inputs(M, E, k, seed=3, device="cuda"),
                    step=lambda x: impl_hip.run(*x), kernel=f"tb::filter_kernel<0, {E // 16}, 8, 1, true>", cpu=cpu)
    return make


def _w_gating_reference_grid():
    import torch
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_hip, impl_torch

    M, E, k = 20480, 128, 2
    nbytes = M * E * 2 + M * k * 2 + M * k * 4       # moe_topk_gating/config.yaml bytes_expr, fp16

    def gen(device):
        return T.generate_moe_topk_gating_inputs(M, E, k, dtype=torch.float16, dist="grid", seed=3, device=device)

    def cpu():
        x = gen("cpu")
        return (lambda: impl_torch.run(*x)), nbytes, "full M = 20480, E = 128, k = 2, fp16"

    return dict(name="moe_topk_gating_ref_grid",
                config={"workload": "moe_topk_gating", "M": M, "E": E, "k": k, "dtype": "fp16", "dist": "grid"},
                metric="MoE gating HBM throughput", unit="GB/s", dtype="fp16", bound="hbm", bytes=nbytes,
                flops=None, out_bytes=M * k * 6, inputs=lambda: gen("cuda"), step=lambda x: impl_hip.run(*x),
                kernel="tb::gating_kernel<1, 16, 8, 2>", cpu=cpu)


def _w_fp8_quant():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.fp8_act_quant import impl_hip, impl_torch

    M = K = 8192
    nbytes = 2 * M * K + M * K + 4 * M

    def cpu():
        x = T.generate_fp8_act_quant_inputs(M, K, seed=2, device="cpu")
        return (lambda: impl_torch.run(*x)), nbytes, "full config 2a (8192 x 8192)"

    return dict(name="fp8_act_quant", config={"workload": "fp8_act_quant", "M": M, "K": K},
                metric="fp8 per-token quant HBM throughput", unit="GB/s", dtype="fp16->e4m3", bound="hbm",
                bytes=nbytes, flops=None, out_bytes=M * K + 4 * M,
                inputs=lambda: T.generate_fp8_act_quant_inputs(M, K, seed=2, device="cuda"),
                step=lambda x: impl_hip.run(*x), kernel="tb::fp8_quant_rows<4>", cpu=cpu)


def _w_w4a16(M, layout="rows"):
    def make():
        from tilebench_amd.data import tensors as T
        from tilebench_amd.benchmarks.operators.w4a16_gemm import impl_hip, impl_torch

        K, N, G = 4096, 11008, 128
        flops = 2 * M * K * N
        nbytes = 2 * M * K + K * N // 2 + (K // G) * N * 2 + (K // G) * N // 2 + 2 * M * N
        big = M > 16

        def cpu():
            rows = min(M, 1024)
            x = T.generate_w4a16_gemm_inputs(rows, K, N, G, seed=1, device="cpu", layout=layout)
            work = 2 * rows * K * N if big else nbytes
            return ((lambda: impl_torch.run(*x)), work,
                    f"{rows} of {M} rows (dequantise W, fp32 matmul)" if big else f"full M = {M}")

        config = {"workload": "w4a16_gemm", "M": M, "K": K, "N": N, "group": G, "weight_layout": layout}
        if layout == "slabs":
            # the layout is a weight format converted once at load; the
            # conversion is not part of a step (repack_us reports its cost)
            config["layout_note"] = ("weights converted once to the decode's slab layout "
                                     "(formats.w4a16_to_slabs) before timing, as at model load")
        kernel = ("tb::w4a16::w4a16_prefill" if big else
                  "tb::slabs::slab_decode<8, 4>" if layout == "slabs" else "tb::w4a16::w4a16_decode<false>")
        name = f"w4a16_gemm_M{M}" + ("_slabs" if layout == "slabs" else "")
        return dict(name=name, config=config,
                    metric="W4A16 GEMM throughput" if big else "W4A16 decode GEMM HBM throughput",
                    unit="TFLOP/s" if big else "GB/s", dtype="fp16 x int4 -> fp16 (fp32 acc)",
                    bound="mfma" if big else "hbm", peak_key="fp16", bytes=nbytes, flops=flops, out_bytes=2 * M * N,
                    inputs=lambda: T.generate_w4a16_gemm_inputs(M, K, N, G, seed=1, device="cuda", layout=layout),
                    step=lambda x: impl_hip.run(*x), kernel=kernel, cpu=cpu,
                    extra=(_slab_repack_us if layout == "slabs" else None))
    return make


def _slab_repack_us():
    """Mean time of one conversion of config 1's weights to the slab layout
    (tb_w4a16_repack_slabs, the load-time step the slab lines leave out)."""
    import torch
    from tilebench_amd import formats
    from tilebench_amd.data import tensors as T

    _, p, _, _, _ = T.generate_w4a16_gemm_inputs(1, 4096, 11008, 128, seed=1, device="cuda")
    formats.w4a16_to_slabs(p)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        formats.w4a16_to_slabs(p)
    e1.record()
    torch.cuda.synchronize()
    return {"repack_us": round(e0.elapsed_time(e1) * 100.0, 2)}


def _w_fp8_quant_blocks():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.fp8_act_quant_blocks import impl_hip, impl_torch

    M = K = 8192
    nbytes = 2 * M * K + M * K + 4 * M * (K // 128)

    def cpu():
        x = T.generate_fp8_act_quant_blocks_inputs(M, K, seed=2, device="cpu")
        return (lambda: impl_torch.run(*x)), nbytes, "full 8192 x 8192"

    return dict(name="fp8_act_quant_blocks", config={"workload": "fp8_act_quant_blocks", "M": M, "K": K, "block": 128},
                metric="fp8 per-token 128-channel quant HBM throughput", unit="GB/s", dtype="fp16->e4m3",
                bound="hbm", bytes=nbytes, flops=None, out_bytes=M * K + 4 * M * (K // 128),
                inputs=lambda: T.generate_fp8_act_quant_blocks_inputs(M, K, seed=2, device="cuda"),
                step=lambda x: impl_hip.run(*x), kernel="tb::fp8blk::fp8_quant_blocks<2>", cpu=cpu)


def _w_fp8_gemm():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.fp8_scaled_gemm import impl_hip, impl_torch

    M = N = K = 8192
    flops = 2 * M * N * K
    nbytes = M * K + K * N + 4 * M + 4 * N + 2 * M * N

    def cpu():
        rows = 2048
        x = T.generate_fp8_scaled_gemm_inputs(rows, N, K, seed=2, device="cpu")
        return ((lambda: impl_torch.run(*x)), 2 * rows * N * K,
                f"{rows} of {M} rows (decoded e4m3 operands, fp32 matmul)")

    return dict(name="fp8_scaled_gemm", config={"workload": "fp8_scaled_gemm", "M": M, "N": N, "K": K},
                metric="fp8 row/column-scaled GEMM throughput", unit="TFLOP/s", dtype="e4m3 x e4m3 -> bf16 (fp32 acc)",
                bound="mfma", peak_key="fp8", bytes=nbytes, flops=flops, out_bytes=2 * M * N,
                inputs=lambda: T.generate_fp8_scaled_gemm_inputs(M, N, K, seed=2, device="cuda"),
                step=lambda x: impl_hip.run(*x), kernel="tb::fp8gemm::fp8_gemm_kernel", cpu=cpu)


def _w_fp8_block_gemm():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.fp8_block_scaled_gemm import impl_hip, impl_torch

    M = N = K = 8192
    flops = 2 * M * N * K
    nbytes = M * K + N * K + 4 * M * (K // 128) + 4 * ((N + 127) // 128) * (K // 128) + 2 * M * N

    def cpu():
        rows = 1024
        x = T.generate_fp8_block_scaled_gemm_inputs(rows, N, K, seed=2, device="cpu")
        return ((lambda: impl_torch.run(*x)), 2 * rows * N * K,
                f"{rows} of {M} rows (block-dequantised operands, fp32 matmul)")

    return dict(name="fp8_block_scaled_gemm", config={"workload": "fp8_block_scaled_gemm", "M": M, "N": N, "K": K,
                                                      "block": 128},
                metric="block-scaled fp8 GEMM throughput (128 x 128 weight blocks, per-token 128-channel "
                       "activation blocks)",
                unit="TFLOP/s", dtype="e4m3 x e4m3 -> bf16 (fp32 acc)", bound="mfma", peak_key="fp8", bytes=nbytes,
                flops=flops, out_bytes=2 * M * N,
                inputs=lambda: T.generate_fp8_block_scaled_gemm_inputs(M, N, K, seed=2, device="cuda"),
                step=lambda x: impl_hip.run(*x), kernel="tb::fp8blk::fp8_block_gemm<256, 8, 2>", cpu=cpu)


def _w_grouped():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.moe_w4a16_grouped_gemm import impl_hip, impl_torch

    tokens, topk, E, K, N, G = 16384, 8, 64, 4096, 1408, 128
    flops = 2 * tokens * topk * K * N
    nbytes = 2 * tokens * topk * K + E * (K * N // 2 + (K // G) * N * 2 + (K // G) * N // 2) + 2 * tokens * topk * N

    def cpu():
        t = 1024
        x = T.generate_moe_w4a16_grouped_gemm_inputs(t, topk, E, K, N, G, seed=4, device="cpu")
        return ((lambda: impl_torch.run(*x)), 2 * t * topk * K * N,
                f"{t} of 16384 tokens x top-8 over all 64 experts (dequantise each W, fp32 matmul)")

    return dict(name="moe_w4a16_grouped_gemm",
                config={"workload": "moe_w4a16_grouped_gemm", "tokens": tokens, "topk": topk, "experts": E, "K": K,
                        "N": N, "group": G, "zipf_s": 1.1, "pad": 128},
                metric="MoE grouped W4A16 GEMM throughput", unit="TFLOP/s", dtype="fp16 x int4 -> fp16 (fp32 acc)",
                bound="mfma", peak_key="fp16", bytes=nbytes, flops=flops, out_bytes=2 * (tokens * topk + E * 128) * N,
                inputs=lambda: T.generate_moe_w4a16_grouped_gemm_inputs(tokens, topk, E, K, N, G, seed=4,
                                                                       device="cuda"),
                step=lambda x: impl_hip.run(*x), kernel="tb::w4a16::w4a16_grouped", cpu=cpu)


def _w_fused_moe():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.fused_moe_w4a16 import impl_hip, impl_torch

    tokens, E, topk, H, I, G13, G2 = 16384, 64, 8, 4096, 704, 128, 64
    flops = 6 * tokens * topk * H * I           # gate/up 2*T*k*H*2I + down 2*T*k*I*H
    wbytes = E * (H * I + (H // G13) * 2 * I * 2 + (H // G13) * I + I * H // 2 + (I // G2) * H * 2 + (I // G2) * H // 2)
    nbytes = 2 * tokens * H + 4 * tokens * E + wbytes + 2 * tokens * H

    def cpu():
        t = 256
        x = T.generate_fused_moe_w4a16_inputs(t, E, topk, H, I, G13, G2, seed=15, device="cpu")
        return ((lambda: impl_torch.run(*x)), 6 * t * topk * H * I,
                f"{t} of 16384 tokens through the whole layer, all 64 experts")

    return dict(name="fused_moe_w4a16",
                config={"workload": "fused_moe_w4a16", "tokens": tokens, "experts": E, "topk": topk, "H": H, "I": I,
                        "group13": G13, "group2": G2, "zipf_s": 1.1},
                metric="MoE layer (gating + sort + W4A16 gate/up + SiLU + W4A16 down + combine) throughput",
                unit="TFLOP/s", dtype="fp16 x int4 -> fp16 (fp32 acc)", bound="mfma", peak_key="fp16",
                bytes=nbytes, flops=flops, out_bytes=2 * tokens * H,
                inputs=lambda: T.generate_fused_moe_w4a16_inputs(tokens, E, topk, H, I, G13, G2, seed=15,
                                                                device="cuda"),
                step=lambda x: impl_hip.run(*x), kernel="tb::w4a16::moe_gate_up", cpu=cpu)


def _w_weight_dequant():
    import torch
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.weight_dequant import impl_hip, impl_torch

    M, TS = 10240, 128
    nbytes = 2 * M * M * 2 + ((M + TS - 1) // TS) ** 2 * 2   # weight_dequant/config.yaml bytes_expr, fp16

    def cpu():
        rows = 1024
        x = T.generate_weight_dequant_inputs(rows, TS, dtype=torch.float16, N=M, seed=10, device="cpu")
        return (lambda: impl_torch.run(*x)), 4 * rows * M, f"{rows} of {M} rows, fp16"

    return dict(name="weight_dequant", config={"workload": "weight_dequant", "M": M, "TILE_SIZE": TS, "dtype": "fp16"},
                metric="weight_dequant HBM throughput", unit="GB/s", dtype="fp16", bound="hbm", bytes=nbytes,
                flops=M * M, out_bytes=2 * M * M,
                inputs=lambda: T.generate_weight_dequant_inputs(M, TS, dtype=torch.float16, seed=10, device="cuda"),
                step=lambda x: impl_hip.run(*x), kernel="tb::analog::weight_dequant_vec<1>", cpu=cpu)


def _w_dequantize_rowwise():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.dequantize_rowwise import impl_hip, impl_torch

    rows, cols = 4096, 8192
    nbytes = rows * cols + rows * 4 + rows * cols * 2            # dequantize_rowwise/config.yaml bytes_expr

    def cpu():
        x = T.generate_dequantize_rowwise_inputs(rows, cols, seed=11, device="cpu")
        return (lambda: impl_torch.run(*x)), nbytes, "full 4096 x 8192"

    return dict(name="dequantize_rowwise", config={"workload": "dequantize_rowwise", "rows": rows, "cols": cols},
                metric="dequantize_rowwise HBM throughput", unit="GB/s", dtype="int8->fp16", bound="hbm",
                bytes=nbytes, flops=2 * rows * cols, out_bytes=2 * rows * cols,
                inputs=lambda: T.generate_dequantize_rowwise_inputs(rows, cols, seed=11, device="cuda"),
                step=lambda x: impl_hip.run(*x), kernel="tb::analog::dequant_rowwise_rows", cpu=cpu)


def _w_quantize_global():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.quantize_global import impl_hip, impl_torch

    n = 20 * 1024 * 1024
    nbytes = n * 4 + n * 2

    def cpu():
        x = T.generate_quantize_global_inputs(n, seed=12, device="cpu")
        return (lambda: impl_torch.run(*x)), nbytes, "full n = 20 Mi"

    return dict(name="quantize_global", config={"workload": "quantize_global", "n": n},
                metric="quantize_global HBM throughput", unit="GB/s", dtype="fp32->fp16", bound="hbm", bytes=nbytes,
                flops=None, out_bytes=2 * n, inputs=lambda: T.generate_quantize_global_inputs(n, seed=12, device="cuda"),
                step=lambda x: impl_hip.run(*x), kernel="tb::analog::f32_to_f16_vec", cpu=cpu)


def _w_matmul_int8():
    from tilebench_amd.data import tensors as T
    from tilebench_amd.benchmarks.operators.matmul_int8 import impl_hip, impl_torch

    M = N = 2048
    K = 20480
    nbytes = M * K + K * N // 4 + 4 * M * N          # matmul_int8/config.yaml bytes_expr

    def cpu():
        rows = 256
        a, b = T.generate_matmul_int8_inputs(M, N, K, seed=13, device="cpu")
        a = a[:rows].contiguous()
        return (lambda: impl_torch.run(a, b)), 2 * rows * N * K, f"{rows} of {M} rows (fp32 matmul, exact)"

    return dict(name="matmul_int8", config={"workload": "matmul_int8", "M": M, "N": N, "K": K},
                metric="matmul_int8 throughput", unit="TFLOP/s", dtype="int8 x int2 -> int32", bound="mfma",
                peak_key="int8", bytes=nbytes, flops=2 * M * N * K, out_bytes=4 * M * N,
                inputs=lambda: T.generate_matmul_int8_inputs(M, N, K, seed=13, device="cuda"),
                step=lambda x: impl_hip.run(*x), kernel="tb::ntg::nt_gemm<3, 4, 256, 256, 128, 64>", cpu=cpu)


def _w_matmul(dt):
    def make():
        import torch
        from tilebench_amd.data import tensors as T
        from tilebench_amd.benchmarks.operators.matmul_fp32_fp16_fp8 import impl_hip, impl_torch

        M = N = 4096
        K = 20480
        tdt = {"fp32": torch.float32, "fp16": torch.float16, "fp8_e4m3fn": torch.float8_e4m3fn}[dt]
        esz = {"fp32": 4, "fp16": 2, "fp8_e4m3fn": 1}[dt]
        nbytes = (M * K + K * N + M * N) * esz          # matmul_fp32_fp16_fp8/config.yaml bytes_expr

        def cpu():
            rows = 64
            a, b = T.generate_matmul_fp32_fp16_fp8_inputs(M, N, K, dtype=tdt, seed=14, device="cpu")
            a = a[:rows].contiguous()
            return (lambda: impl_torch.run(a, b)), 2 * rows * N * K, f"{rows} of {M} rows"

        kern = {"fp32": "tb::ntg::nt_gemm<2, 3, 256, 256, 128, 64>", "fp16": "tb::ntg::nt_gemm<1, 2, 256, 256, 128, 64>",
                "fp8_e4m3fn": "tb::ntg::nt_gemm<0, 1, 256, 256, 128, 64>"}[dt]
        w = dict(name=f"matmul_{dt}", config={"workload": "matmul_fp32_fp16_fp8", "M": M, "N": N, "K": K, "dtype": dt},
                 metric="matmul throughput", unit="TFLOP/s", dtype=dt, bound="mfma",
                 peak_key={"fp32": "bf16", "fp16": "fp16", "fp8_e4m3fn": "fp8"}[dt], bytes=nbytes,
                 flops=2 * M * N * K, out_bytes=M * N * esz,
                 inputs=lambda: T.generate_matmul_fp32_fp16_fp8_inputs(M, N, K, dtype=tdt, seed=14, device="cuda"),
                 step=lambda x: impl_hip.run(*x), kernel=kern, cpu=cpu)
        if dt == "fp32":
            # computed as one bf16 GEMM over 3K (hi*hi + hi*lo + lo*hi): the matrix
            # pipe does 3x the fp32 product's flops, priced against the bf16 peak
            w["dtype"] = "fp32 (3 x bf16 products, fp32 acc)"
            w["mfma_flops"] = 3 * 2 * M * N * K
        return w
    return make


def _w_copy():
    import torch

    nbytes = 1 << 30

    def step(x):
        from tilebench_amd import runtime as rt
        src = x[0]
        dst = torch.empty_like(src)
        rt.call("tb_probe_copy", src.data_ptr(), dst.data_ptr(), src.numel(), rt.stream_handle())
        return dst

    return dict(name="hbm_copy_probe", config={"workload": "hbm_copy_probe", "bytes": nbytes},
                metric="HBM streaming copy (calibration probe)", unit="GB/s", dtype="u8", bound="hbm", bytes=nbytes,
                flops=None, out_bytes=nbytes // 2,
                inputs=lambda: (torch.empty(nbytes // 2, dtype=torch.uint8, device="cuda"),), step=step,
                kernel="tb::copy_kernel", cpu=None)


WORKLOADS = {
    "w4a16_gemm_M4096": _w_w4a16(4096),
    "w4a16_gemm_M16": _w_w4a16(16),
    "w4a16_gemm_M1": _w_w4a16(1),
    "w4a16_gemm_M16_slabs": _w_w4a16(16, "slabs"),
    "w4a16_gemm_M1_slabs": _w_w4a16(1, "slabs"),
    "int4_dequant": _w_int4_dequant,
    "moe_topk_gating_E64": _w_gating(64),
    "moe_topk_gating_E256": _w_gating(256),
    "moe_topk_gating_ref_grid": _w_gating_reference_grid,
    "fp8_act_quant": _w_fp8_quant,
    "fp8_scaled_gemm": _w_fp8_gemm,
    "fp8_block_scaled_gemm": _w_fp8_block_gemm,
    "fp8_act_quant_blocks": _w_fp8_quant_blocks,
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
#: every BASELINE config besides the headline: measured in the default line's `suite`
BASELINE_SUITE = ("int4_dequant", "w4a16_gemm_M1", "w4a16_gemm_M16", "w4a16_gemm_M1_slabs", "w4a16_gemm_M16_slabs",
                  "fp8_act_quant", "fp8_scaled_gemm", "moe_topk_gating_E64", "moe_topk_gating_E256",
                  "moe_w4a16_grouped_gemm", "fp8_block_scaled_gemm")


# ----------------------------------------------------------------------------- measurement


def _footprint(x) -> int:
    import torch
    return sum(t.numel() * t.element_size() for t in x if isinstance(t, torch.Tensor))


def input_sets(w, x, steps: int) -> tuple[list, list]:
    """Device copies of the inputs at distinct addresses: (timed sets, warm sets).

    A step moves its inputs plus its output (`traffic`).  With n =
    ceil(2 x MALL / traffic) + 1 sets cycling, a set is used again after the
    n - 1 steps on the other sets, which move at least 2x the MALL of other
    traffic in between (the reference evicts the LLC before every timed
    launch, tilebench/core/timer.py:81-117, with a 2 x LLC flush).  The timed
    graph cycles over min(steps, n) sets (with steps < n no set is used twice);
    the warm graph and the eager warmup cycle over n further sets, so when the
    timed replay starts its sets have not been touched for at least 2x the MALL
    of traffic either."""
    import torch
    traffic = _footprint(x) + w.get("out_bytes", 0)
    n = 1 + max(1, -(-2 * MALL_BYTES // max(traffic, 1)))
    n_timed = min(steps, n)
    sets = [x] + [tuple(t.clone() if isinstance(t, torch.Tensor) else t for t in x) for _ in range(n_timed + n - 1)]
    return sets[:n_timed], sets[n_timed:]


def _capture(w, sets, steps):
    import torch
    graph = torch.cuda.CUDAGraph()
    keep = []
    with torch.cuda.graph(graph):
        for i in range(steps):
            keep.append(w["step"](sets[i % len(sets)]))  # outputs: a ring of 8 fresh allocations
            if len(keep) > 8:
                keep.pop(0)
    return graph, keep


def time_steps(w, timed, warm, steps: int, warmup: int) -> dict:
    """Mean ms per step of `steps` launches in one timed graph replay (see the
    module docstring), and how the region was prepared."""
    import torch

    for i in range(max(1, warmup)):
        w["step"](warm[i % len(warm)])
    # one eager step on every input set before capture (no operator keeps
    # per-input state; this touches every set once, as the timed replay will)
    for x in list(timed) + list(warm):
        w["step"](x)
    torch.cuda.synchronize()
    g_warm, keep_w = _capture(w, warm, steps)
    g_timed, keep_t = _capture(w, timed, steps)
    g_timed.replay()  # uploads the timed graph; its sets are then evicted by the warm replays below
    stream = torch.cuda.current_stream()
    # One warm replay, timed, sizes the warm phase: at least 2x the MALL of
    # traffic (the eviction above) and at least WARM_MS of back-to-back work, so
    # the timed replay runs at the clock the GPU holds under sustained load
    # whatever K is (a 20-step replay of a 0.3 ms kernel alone is 6 ms).
    w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0.record(stream)
    g_warm.replay()
    w1.record(stream)
    torch.cuda.synchronize()
    per_replay = max(w0.elapsed_time(w1), 1e-3)
    traffic = (_footprint(timed[0]) + w.get("out_bytes", 0)) * steps
    warm_replays = max(1, -(-2 * MALL_BYTES // max(traffic, 1)), math.ceil(WARM_MS / per_replay))
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(warm_replays):
        g_warm.replay()
    start.record(stream)
    g_timed.replay()
    stop.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    del keep_w, keep_t, g_warm, g_timed
    return {"ms": ms, "untimed_replays_before": warm_replays, "warm_ms": round(warm_replays * per_replay, 1),
            "timed_sets": len(timed), "warm_sets": len(warm)}


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

#: the calibration protocol, shortened for a live measurement inside the bench
LIVE_PROTOCOL = {"batches": 3, "warmup": 3, "repeat": 5, "target_sample_ms": 2.0}


def measured_peak(bound: str, peak_key: str | None):
    """The peak this GPU reaches now, in this process, by the calibration
    protocol (tilebench_amd/calibration.py: median over 3 batches of each
    batch's median sample): HBM GB/s from tb_probe_copy over 1 GiB each way (a
    2 GiB working set, 8x the MALL); matrix TFLOP/s from tb_probe_mfma (8
    independent 32x32 MFMA chains per wavefront, two 4-wavefront blocks per
    CU).  Measured once per process per key."""
    import torch
    from tilebench_amd import calibration as cal
    from tilebench_amd import runtime as rt

    key = "hbm" if bound == "hbm" else peak_key
    if key in _MEASURED_PEAKS:
        return _MEASURED_PEAKS[key]
    kinds = {"fp16": (0, 32768), "fp8": (1, 131072), "bf16": (2, 32768), "int8": (3, 65536)}
    stream = rt.stream_handle()
    if key == "hbm":
        n = 1 << 30
        src = torch.empty(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        fn = lambda: rt.call("tb_probe_copy", src.data_ptr(), dst.data_ptr(), n, stream)  # noqa: E731
        work, scale = 2 * n, 1e9
    elif key in kinds:
        kind, per = kinds[key]
        blocks, iters = 2 * torch.cuda.get_device_properties(0).multi_processor_count, 2000
        out = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
        fn = lambda: rt.call("tb_probe_mfma", kind, blocks, iters, out.data_ptr(), stream)  # noqa: E731
        work, scale = blocks * 4 * 8 * iters * per, 1e12
    else:
        _MEASURED_PEAKS[key] = None
        return None
    meas = cal.measure(fn, LIVE_PROTOCOL)
    _MEASURED_PEAKS[key] = round(work / (cal.point_time(meas["batches_ms"]) * 1e-3) / scale, 2)
    return _MEASURED_PEAKS[key]


def calibrated_peak(bound: str, peak_key: str | None):
    """The committed calibration (tilebench_amd/data/peak_performance/empirical/
    MI355X.json, written by `python -m tilebench_amd.calibration`) for this
    bound, or None."""
    from tilebench_amd.core.metrics import load_calibrated_peaks

    cfg = load_calibrated_peaks("MI355X")
    if bound == "hbm":
        return cfg.get("peak_bw_GBs")
    ck = CALIBRATION_KEY.get(peak_key or "")
    if ck is None:
        return None
    return {**(cfg.get("peak_tops") or {}), **(cfg.get("peak_tflops") or {})}.get(ck)


def roofline(w, ms: float) -> dict:
    if w["bound"] == "hbm":
        achieved = w["bytes"] / (ms * 1e-3) / 1e9
        peak, unit = PEAK_HBM_GBS, "GB/s"
    else:
        achieved = w.get("mfma_flops", w["flops"]) / (ms * 1e-3) / 1e12
        peak, unit = PEAK_TFLOPS[w["peak_key"]], "TFLOP/s"
    mp = measured_peak(w["bound"], w.get("peak_key"))
    cp = calibrated_peak(w["bound"], w.get("peak_key"))
    out = {"bound": w["bound"], "achieved": round(achieved, 2), "peak": peak, "unit": unit,
           "frac": round(achieved / peak, 4), "traffic": measured_traffic(w["kernel"]),
           "kernel": w["kernel"], "alg_read_bytes": w["bytes"] - w.get("out_bytes", 0),
           "alg_write_bytes": w.get("out_bytes", 0),
           "measured_peak": mp,
           "frac_of_measured": None if mp is None else round(achieved / mp, 4),
           "calibrated_peak": cp, "frac_of_calibrated": None if cp is None else round(achieved / cp, 4)}
    if "mfma_flops" in w:
        out["note"] = (f"achieved counts the bf16 MFMA work ({w['mfma_flops'] / w['flops']:.0f}x the fp32 "
                       f"GEMM's flops); as fp32 work: {w['flops'] / (ms * 1e-3) / 1e12:.2f} TFLOP/s")
    return out


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _host_cores() -> int:
    """The cores this process may run on (the affinity mask, else cpu_count)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_baseline(w, warmup: int = 1, repeat: int = 3) -> dict:
    """The PyTorch CPU reference (impl_torch.run) on the workload's bounded CPU
    sample: warmup 1, repeat 3 timed with perf_counter (the reference protocol,
    tilebench/core/timer.py:43-44), all host cores given to torch."""
    import torch

    prev = torch.get_num_threads()
    cores = _host_cores()
    torch.set_num_threads(cores)
    try:
        fn, work, sample = w["cpu"]()
        for _ in range(warmup):
            fn()
        times = []
        for _ in range(repeat):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        used = torch.get_num_threads()
    finally:
        torch.set_num_threads(prev)
    mean = sum(times) / len(times)
    value = work / mean / (1e9 if w["unit"] == "GB/s" else 1e12)
    return {"value": round(value, 4), "unit": w["unit"], "cores": used, "kind": "port", "impl": "torch",
            "sample": f"impl_torch.run on CPU tensors, {sample}; warmup {warmup}, repeat {repeat}: "
                      f"{', '.join(f'{t * 1e3:.1f}' for t in times)} ms",
            "os_cpu_count": os.cpu_count(), "affinity_cores": cores, "cpu_model": _cpu_model()}


def measure(name: str, steps: int, warmup: int, with_cpu: bool) -> dict:
    import torch

    w = WORKLOADS[name]()
    x = w["inputs"]()
    timed, warm = input_sets(w, x, steps)
    del x
    torch.cuda.synchronize()
    t = time_steps(w, timed, warm, steps, warmup)
    out = {"name": w["name"], "w": w, "ms": t["ms"], "timing": t, "roofline": roofline(w, t["ms"])}
    if w.get("extra"):
        out["extra"] = w["extra"]()
    del timed, warm
    torch.cuda.empty_cache()
    if with_cpu and w.get("cpu"):
        out["cpu_baseline"] = cpu_baseline(w)
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--op", default=DEFAULT_OP, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-suite", action="store_true", help="headline only (no other BASELINE configs)")
    ap.add_argument("--suite", action="store_true", help="also the analog operators, the MoE layer and the copy probe")
    ap.add_argument("--only", default=None, help="comma-separated workloads for the suite (default: see --suite)")
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

    with_cpu = not args.no_cpu_baseline
    main_res = measure(args.op, args.steps, args.warmup, with_cpu)
    w, ms = main_res["w"], main_res["ms"]
    line = {
        "metric": w["metric"], "value": main_res["roofline"]["achieved"], "unit": w["unit"], "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": w["dtype"],
        "data": "synthetic (seeded CPU generator, resident in HBM)",
        "config": {**w["config"], "input_sets": main_res["timing"]["timed_sets"]},
        "timing": {"untimed_replays_before": main_res["timing"]["untimed_replays_before"],
                   "warm_ms": main_res["timing"]["warm_ms"],
                   "warm_sets": main_res["timing"]["warm_sets"],
                   "region": "K steps in one hipGraph replay between hipEvents, after untimed replays of the "
                             "same K steps on other input copies (at least 200 ms of them, no host sync "
                             "between them and the timed replay)"},
        "roofline": main_res["roofline"],
        "cpu_baseline": main_res.get("cpu_baseline"),
    }
    if not args.no_suite:
        if args.only:
            names = args.only.split(",")
        else:
            names = list(BASELINE_SUITE) + ([n for n in WORKLOADS if n not in BASELINE_SUITE] if args.suite else [])
        suite = {}
        for name in names:
            if name == args.op:
                continue
            r = measure(name, args.steps, args.warmup, with_cpu)
            suite[name] = {"metric": r["w"]["metric"], "config": {**r["w"]["config"],
                                                                  "input_sets": r["timing"]["timed_sets"]},
                           "ms": round(r["ms"], 6), "untimed_replays_before": r["timing"]["untimed_replays_before"],
                           **r["roofline"], **(r.get("extra") or {}), "cpu_baseline": r.get("cpu_baseline")}
            print(f"[bench] {name}: {r['ms'] * 1e3:.1f} us/step, {r['roofline']['achieved']} "
                  f"{r['roofline']['unit']}", file=sys.stderr, flush=True)
        line["suite"] = suite
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
