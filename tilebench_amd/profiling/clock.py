"""Shader clock and sample times by what ran just before a launch.

The harness (core.timer) takes each sample of an operator after a host
synchronisation and a 512 MiB flush; bench.py replays K steps back to back
after at least 200 ms of warm replays.  For an MFMA-bound launch of a
millisecond or more the two can disagree by 15-25 %.  This tool separates
the candidate causes:

  part 1, the clock: tb_probe_clock runs fp16 MFMAs on every SIMD for about
  1.5 ms and reports each block's average shader clock (the s_memtime counter
  against the constant 100 MHz one).  Launches back to back, each right after
  a synchronisation, and after a synchronisation plus an idle of 0.5, 2 and
  20 ms.

  part 2, the operator: one hipGraph replay of impl_hip.run on the operator's
  config.yaml defaults, hipEvent-timed, preceded by (a) the synchronisation
  only, (b) the harness's flush (core.timer.flush_l2_cache), (c) the flush and
  an idle of 2 / 20 ms, (d) a 512 MiB read sweep (tb_probe_read, clean lines)
  instead of the flush.  The variants are interleaved over ROUNDS rounds.

Usage:  python -m tilebench_amd.profiling.clock [--operator moe_w4a16_grouped_gemm] [--out FILE]
"""
from __future__ import annotations

import argparse
import importlib
import statistics
import sys
import time

MIB = 1024 * 1024


def _probe_clock(rt, blocks: int, iters: int, clocks, sink) -> None:
    rt.call("tb_probe_clock", blocks, iters, clocks.data_ptr(), sink.data_ptr(), rt.stream_handle())


def _mhz(clocks) -> float:
    c = clocks.view(-1, 2).double().cpu()
    return float((c[:, 0] / c[:, 1]).mean() * 100.0)


def clock_part(rt, torch, blocks: int = 1024, target_ms: float = 1.5) -> list[str]:
    sink = torch.empty(blocks * 4, device="cuda")
    bufs = [torch.zeros(blocks * 2, dtype=torch.int64, device="cuda") for _ in range(20)]
    # size the loop so one launch takes about target_ms
    iters = 200
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(3):
        _probe_clock(rt, blocks, iters, bufs[0], sink)
    e0.record()
    _probe_clock(rt, blocks, iters, bufs[0], sink)
    e1.record()
    torch.cuda.synchronize()
    iters = max(1, int(iters * target_ms / e0.elapsed_time(e1)))
    out = [f"part 1: tb_probe_clock, {blocks} blocks x 256 threads, {iters} iterations of 8 fp16 MFMAs "
           f"(about {target_ms} ms per launch)"]
    for i in range(20):
        _probe_clock(rt, blocks, iters, bufs[i], sink)
    torch.cuda.synchronize()
    out.append("  20 launches back to back, MHz: " + " ".join(f"{_mhz(b):.0f}" for b in bufs))
    for idle in (0.0, 0.0005, 0.002, 0.02):
        mhz, us = [], []
        for i in range(8):
            torch.cuda.synchronize()
            if idle:
                time.sleep(idle)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            _probe_clock(rt, blocks, iters, bufs[i], sink)
            b.record()
            torch.cuda.synchronize()
            mhz.append(_mhz(bufs[i]))
            us.append(a.elapsed_time(b) * 1e3)
        out.append(f"  after sync + {idle * 1e3:4.1f} ms idle: MHz " + " ".join(f"{m:.0f}" for m in mhz) +
                   "  | us " + " ".join(f"{u:.0f}" for u in us))
    return out


def operator_part(rt, torch, operator: str, rounds: int = 6) -> list[str]:
    import yaml

    from tilebench_amd.core import timer
    from tilebench_amd.core.dtypes import resolve_dtype
    from tilebench_amd.data.tensors import get_generator
    from tilebench_amd.paths import operator_config

    cfg = yaml.safe_load(open(operator_config(operator)))
    params = dict(cfg.get("case_defaults") or {})
    dtype = params.pop("dtype", None) or (cfg.get("case_grid") or {}).get("dtype", ["fp16"])[0]
    impl = importlib.import_module(f"tilebench_amd.benchmarks.operators.{operator}.impl_hip")
    x = get_generator(operator)(**params, dtype=resolve_dtype(dtype))
    for _ in range(2):
        impl.run(*x)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        impl.run(*x)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=side):
            impl.run(*x)
    torch.cuda.synchronize()
    clean = torch.zeros(512 * MIB, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")

    def read_sweep():
        rt.call("tb_probe_read", clean.data_ptr(), clean.numel(), 0xDEADBEEF, sink.data_ptr(), rt.stream_handle())

    variants = {"sync only": (lambda: None, 0.0), "flush": (timer.flush_l2_cache, 0.0),
                "flush + 2 ms idle": (timer.flush_l2_cache, 0.002), "flush + 20 ms idle": (timer.flush_l2_cache, 0.02),
                "512 MiB read instead": (read_sweep, 0.0)}
    res = {k: [] for k in variants}
    for _ in range(rounds):
        for k, (pre, idle) in variants.items():
            pre()
            torch.cuda.synchronize()
            if idle:
                time.sleep(idle)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            g.replay()
            b.record()
            torch.cuda.synchronize()
            res[k].append(a.elapsed_time(b) * 1e3)
    out = [f"part 2: {operator} ({', '.join(f'{k}={v}' for k, v in params.items())}), one graph replay per sample, "
           f"{rounds} rounds of the variants interleaved; hipEvent us"]
    for k, v in res.items():
        out.append(f"  {k:22s} median {statistics.median(v):9.1f}  min {min(v):9.1f}  max {max(v):9.1f}")
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--operator", default="moe_w4a16_grouped_gemm", help="operator for part 2 (empty: skip)")
    ap.add_argument("--out", default=None, help="also write the report here")
    args = ap.parse_args(argv)
    import torch

    if not torch.cuda.is_available():
        print("the clock probe needs a GPU", file=sys.stderr)
        return 2
    from tilebench_amd import runtime as rt

    rt.require_device()
    rt.load_library()
    lines = clock_part(rt, torch)
    for ln in lines:
        print(ln, flush=True)
    if args.operator:
        more = operator_part(rt, torch, args.operator)
        for ln in more:
            print(ln, flush=True)
        lines += more
    if args.out:
        with open(args.out, "w") as f:
            f.write("\n".join(lines) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
