"""Command line of the harness: run one operator's cases through the engine.

    python -m tilebench_amd.run_bench --operator int4_dequant [--tile-language hip]
        [--grid reference] [--case-indices 0,2] [--warmup W] [--repeat R]
        [--no-flush-l2] [--output results.json]

The counterpart of the reference's scripts/run_bench.py (its --operator,
--tile-language, --case-indices, --warmup, --repeat and --flush-l2 options)
for the backends this package ships: for each case it generates the inputs,
runs the torch reference, then runs, verifies and times the selected
backends (tilebench_amd.core.engine.run_benchmark_suite with the real
hipGraph/hipEvent timer), and prints one line per case with the derived
metrics: % of the device's published peaks (pct_peak_*, the reference's
definition) and of the peaks calibrated on the box (pct_calibrated_peak_*).
"""
from __future__ import annotations

import argparse
import json
import math
import sys

from tilebench_amd.backends import parse_backends


def _fmt(v, spec=".4f"):
    return "nan" if v is None or (isinstance(v, float) and math.isnan(v)) else format(v, spec)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--operator", required=True)
    ap.add_argument("--tile-language", default="hip", help="backends to run besides torch (default: hip)")
    ap.add_argument("--grid", default=None, help="a named grid of the operator's config.yaml (e.g. reference)")
    ap.add_argument("--case-indices", default=None, help="comma-separated case indices")
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--repeat", type=int, default=None)
    ap.add_argument("--no-flush-l2", action="store_true")
    ap.add_argument("--output", default=None, help="write the result rows (JSON) here")
    args = ap.parse_args(argv)

    import torch
    import yaml

    if not torch.cuda.is_available():
        print("run_bench needs a GPU", file=sys.stderr)
        return 2
    from tilebench_amd.core import engine, metrics
    from tilebench_amd.paths import operator_config

    over = {}
    if args.grid:
        over["grid"] = args.grid
    if args.case_indices:
        over["case_indices"] = [int(i) for i in args.case_indices.split(",")]
    if args.warmup is not None:
        over["warmup"] = args.warmup
    if args.repeat is not None:
        over["repeat"] = args.repeat
    if args.no_flush_l2:
        over["flush_l2"] = False
    backends = parse_backends(args.tile_language)
    rows = engine.run_benchmark_suite(args.operator, benchmark_overrides=over, enabled_backends=backends)
    cfg = yaml.safe_load(open(operator_config(args.operator)))
    from tilebench_amd import calibration
    gpu = calibration.gpu_model(calibration.environment())
    peak, calibrated = metrics.load_peak_config(gpu), metrics.load_calibrated_peaks(gpu)
    print(f"# {gpu}: % of peak against {'the published peaks' if peak else 'no published peak file'}"
          f"{', pct_calibrated_* against the calibrated peaks' if calibrated else ''}", flush=True)
    for r in rows:
        r["derived"] = metrics.compute_derived(r, cfg.get("metrics", {}), peak, calibrated)
        line = [f"{k}={v}" for k, v in r["params"].items()] + [f"dtype={r['dtype']}",
                                                                 f"torch_ms={_fmt(r['torch_ms'])}"]
        for b in backends:
            d = r["derived"].get(b, {})
            line += [f"{b}_ok={r[f'{b}_ok']}", f"{b}_ms={_fmt(r[f'{b}_ms'])}"]
            st = r.get(f"{b}_stats") or {}
            if st:
                line += [f"{b}_event_ms={_fmt(st.get('event_mean'))}", f"{b}_time={st.get('time_source')}"]
            if "bandwidth_GBs" in d:
                line.append(f"{b}_GBs={_fmt(d['bandwidth_GBs'], '.1f')}")
            if "tflops" in d:
                line.append(f"{b}_TFLOPS={_fmt(d['tflops'], '.1f')}")
            for key in ("pct_peak_bw", "pct_peak_tflops", "pct_calibrated_peak_bw", "pct_calibrated_peak_tflops"):
                if key in d:
                    line.append(f"{b}_{key}={_fmt(d[key], '.1f')}")
            if not r[f"{b}_ok"]:
                line.append(f"{b}_err={r[f'{b}_err']!r}")
        print("  ".join(line), flush=True)
    if args.output:
        with open(args.output, "w") as f:
            json.dump(rows, f, indent=1, default=str)
    return 0 if all(r[f"{b}_ok"] for r in rows for b in backends) else 1


if __name__ == "__main__":
    sys.exit(main())
