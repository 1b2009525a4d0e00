"""Benchmark of the hip backend's hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--op NAME] [--no-cpu-baseline]

A step is one launch of the operator on one batch of seeded synthetic input
already resident in HBM.  W untimed warmup steps, then exactly K steps between
two hipEvents on the stream the kernels run on (bracketed by
torch.cuda.synchronize()).  Prints ONE JSON line with the driver's fields plus:

  roofline      achieved GB/s or TFLOP/s of the operator's kernel (algorithmic
                bytes or flops per launch / mean launch time from the events),
                MI355X's published peak and the fraction;
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

# MI355X published peaks (dense): HBM3E 8 TB/s; MFMA fp16/bf16 2.5 PFLOP/s, fp8 5.0 PFLOP/s.
PEAK_HBM_GBS = 8000.0
PEAK_TFLOPS = {"fp16": 2500.0, "bf16": 2500.0, "fp8": 5000.0}


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
                kernel="int4_dequant_vec", cpu_sample=cpu_sample)


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
                    flops=None, inputs=inputs, step=lambda x: impl_hip.run(*x), kernel="gating_kernel",
                    cpu_sample=cpu_sample)
    return make


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
                bytes=nbytes, flops=None, inputs=inputs, step=lambda x: impl_hip.run(*x), kernel="fp8_quant_rows",
                cpu_sample=cpu_sample)


WORKLOADS = {
    "int4_dequant": _w_int4_dequant,
    "moe_topk_gating_E64": _w_gating(64),
    "moe_topk_gating_E256": _w_gating(256),
    "fp8_act_quant": _w_fp8_quant,
}
DEFAULT_OP = "int4_dequant"


# ----------------------------------------------------------------------------- measurement

def time_steps(w, x, steps: int, warmup: int):
    """Mean ms per step over `steps` back-to-back launches (events on the launch stream)."""
    import torch

    for _ in range(warmup):
        w["step"](x)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(steps):
        w["step"](x)
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def roofline(w, ms: float) -> dict:
    if w["bound"] == "hbm":
        achieved = w["bytes"] / (ms * 1e-3) / 1e9
        peak, unit = PEAK_HBM_GBS, "GB/s"
    else:
        achieved = w["flops"] / (ms * 1e-3) / 1e12
        peak, unit = PEAK_TFLOPS[w["peak_key"]], "TFLOP/s"
    return {"bound": w["bound"], "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": w.get("traffic")}


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
    x = w["inputs"]()
    torch.cuda.synchronize()
    ms = time_steps(w, x, steps, warmup)
    out = {"name": w["name"], "w": w, "ms": ms, "roofline": roofline(w, ms)}
    if with_cpu:
        out["cpu_baseline"] = cpu_baseline(w)
    del x
    torch.cuda.empty_cache()
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--op", default=DEFAULT_OP, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--suite", action="store_true", help="also measure every other workload")
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
        "config": w["config"], "roofline": main_res["roofline"],
        "cpu_baseline": main_res.get("cpu_baseline"),
    }
    if args.suite:
        suite = {}
        for name in WORKLOADS:
            if name == args.op:
                continue
            r = measure(name, args.steps, args.warmup, False)
            suite[name] = {"ms": round(r["ms"], 6), **r["roofline"]}
        line["suite"] = suite
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
