"""Kernel launches of ONE impl_hip.run() per (operator, dtype), the hip
backend's counterpart of the reference's scripts/profiling/probe_kernel_count.py.

For every operator and dtype of its case grid: generate the inputs of the
sweep-max case (the largest problem of that dtype, as the reference probes
the catalogue's default case), record the first call (library loaded, caches
cold) and a later call under torch.profiler, and keep the device-launch
sequence of each.  One row per pair, with the reference's keys:

    {"op", "dtype", "backend": "hip", "params",
     "count":    backend kernel launches of ONE run(), repeats kept,
     "names":    those launches in launch order (the stems the profilers print),
     "excluded": every other device launch of the call (ATen helpers, runtime
                 copies and fills),
     "first_call_identical": whether the first call launched the same sequence,
     "first_call_names": the first call's backend launches}

With ``--all-cases`` every case of the grid is probed, and each row also lists
the distinct launch sequences with the cases that produce them (the hip
backend picks its kernels by shape: decode or prefill, tile size, a transpose
fallback for odd widths); the operator's named grids (config.yaml "grids:", as
``run_bench --grid`` runs them) get one row each, {"op", "grid", "backend",
"cases", "sequences"}.  A failed probe records count=None and the error.

Usage:  python -m tilebench_amd.profiling.probe --out profiles/kernel_counts_hip_MI355X.json
        python -m tilebench_amd.profiling.probe --ops w4a16_gemm,matmul_int8 --all-cases
"""
from __future__ import annotations

import argparse
import importlib
import inspect
import json
import sys
from pathlib import Path

import torch
import yaml

from tilebench_amd.core.dtypes import resolve_dtype
from tilebench_amd.data.tensors import expand_cases, get_generator, infer_problem_size
from tilebench_amd.paths import list_operators, operator_config
from tilebench_amd.profiling import kernels as kn


def device_launches(prof) -> list[str]:
    """Device launches recorded by torch.profiler, in launch order (HIP kernels
    are reported under DeviceType.CUDA on ROCm)."""
    evs = [e for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]
    evs.sort(key=lambda e: e.time_range.start)
    return [e.key for e in evs]


def _call(impl, inputs, kw):
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
        impl.run(*inputs, **kw)
        torch.cuda.synchronize()
    return device_launches(prof)


def _run_kwargs(fn, case):
    sig = inspect.signature(fn).parameters
    return {"block_size": case["block_size"]} if "block_size" in sig and "block_size" in case else {}


def probe_case(impl, op: str, case: dict) -> dict:
    params = {k: v for k, v in case.items() if k not in ("dtype", "block_size")}
    inputs = get_generator(op)(**params, dtype=resolve_dtype(case.get("dtype", "fp32")))
    if not isinstance(inputs, tuple):
        inputs = (inputs,)
    kw = _run_kwargs(impl.run, case)
    torch.cuda.synchronize()
    first = _call(impl, inputs, kw)
    launches = _call(impl, inputs, kw)
    names = [kn.kernel_stem(n) for n in launches if not kn.is_aux_kernel(n)]
    first_names = [kn.kernel_stem(n) for n in first if not kn.is_aux_kernel(n)]
    del inputs
    return {"count": len(names), "names": names,
            "excluded": [n for n in launches if kn.is_aux_kernel(n)],
            "first_call_identical": first_names == names, "first_call_names": first_names}


def probe_operator(op: str, all_cases: bool = False) -> list[dict]:
    impl = importlib.import_module(f"tilebench_amd.benchmarks.operators.{op}.impl_hip")
    with open(operator_config(op)) as fh:
        cfg = yaml.safe_load(fh)
    cases = expand_cases(op, cfg)
    rows = []
    for dt in sorted({str(c.get("dtype", "fp32")) for c in cases}):
        mine = [c for c in cases if str(c.get("dtype", "fp32")) == dt]
        top = max(mine, key=lambda c: infer_problem_size(op, c))
        row = {"op": op, "dtype": dt, "backend": "hip",
               "params": {k: v for k, v in top.items() if k != "dtype"}}
        try:
            row.update(probe_case(impl, op, top))
        except Exception as e:  # a failing pair is recorded, the others still run
            row.update({"count": None, "error": f"{type(e).__name__}: {e}"[:200]})
        if all_cases:
            row["sequences"] = _sequences(impl, op, mine)
        rows.append(row)
        torch.cuda.empty_cache()
    if all_cases:
        # the operator's named grids (config "grids:"), as the engine's --grid runs them
        for name, alt in sorted((cfg.get("grids") or {}).items()):
            gcfg = {k: v for k, v in cfg.items() if k not in ("case_grid", "case_defaults", "test_cases")}
            gcfg.update(alt)
            gcases = expand_cases(op, gcfg)
            rows.append({"op": op, "grid": name, "backend": "hip", "cases": len(gcases),
                         "sequences": _sequences(impl, op, gcases)})
            torch.cuda.empty_cache()
    return rows


def _sequences(impl, op: str, cases: list[dict]) -> list[dict]:
    """Cases grouped by the kernel sequence one call launches."""
    seqs: dict[tuple, list] = {}
    for c in cases:
        p = {k: v for k, v in c.items() if k != "dtype"}
        try:
            key = tuple(probe_case(impl, op, c)["names"])
        except Exception as e:
            key = ("error: " + f"{type(e).__name__}: {e}"[:160],)
        seqs.setdefault(key, []).append(p)
    return [{"names": list(k), "cases": v} for k, v in seqs.items()]


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Probe the hip backend's kernel launches per impl_hip.run().")
    ap.add_argument("--ops", default=None, help="comma-separated operators (default: all)")
    ap.add_argument("--all-cases", action="store_true", help="also probe every case of each grid")
    ap.add_argument("--out", default=None, help="JSON file to write; rows of other operators are kept")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("error: the probe launches the hip kernels and needs a GPU", file=sys.stderr)
        return 2
    ops = args.ops.split(",") if args.ops else list_operators()
    rows = []
    for op in ops:
        print(f"probe {op}", flush=True)
        rows += probe_operator(op, args.all_cases)
    def key(r):  # a dtype row of the default grid, or a named grid's row
        return (r["op"], r.get("dtype") or "grid:" + r["grid"])

    if args.out:
        out = Path(args.out)
        if out.exists():
            probed = {key(r) for r in rows}
            rows += [r for r in json.loads(out.read_text()) if key(r) not in probed]
        rows.sort(key=key)
        out.parent.mkdir(parents=True, exist_ok=True)
        out.write_text(json.dumps(rows, indent=1) + "\n")
    print(f"{'op':26s} {'dtype':11s} {'count':>5s}  first  names")
    for r in rows:
        if "grid" in r:
            for sq in r["sequences"]:
                print(f"{r['op']:26s} {'grid ' + r['grid']:11s} {len(sq['cases']):>5d}  cases  "
                      f"{', '.join(sq['names'])[:100]}")
            continue
        print(f"{r['op']:26s} {r['dtype']:11s} {str(r['count']):>5s}  {str(r.get('first_call_identical')):5s}  "
              f"{', '.join(r.get('names') or [r.get('error', '')])[:100]}")
    failed = [r for r in rows if ("grid" not in r and r["count"] is None) or
              any(sq["names"][0].startswith("error:") for sq in r.get("sequences") or [])]
    return 0 if not failed else 1


if __name__ == "__main__":
    sys.exit(main())
