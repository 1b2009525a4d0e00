"""Kernel durations from rocprofv3 kernel traces of bench.py and of the harness.

    cd /tmp && rocprofv3 --kernel-trace --stats --output-format csv -d OUT -o bench -- \\
        python3 $REPO/bench.py --suite --no-cpu-baseline --steps 20 --warmup 5 > OUT/bench.json
    python -m tilebench_amd.profiling.suite_trace suite OUT OUT/bench.json

    python -m tilebench_amd.profiling.suite_trace launches OUT --kernel REGEX
        every launch of the hip backend's kernels (tb::) whose name matches, in
        trace order: start (us from the first such launch), duration, and the
        kernel that ran just before it with the idle gap in between

bench.py measures its workloads one after another (the headline first, then
the suite in the order of its JSON line), and each workload's graph capture
leaves a block of torch fill launches (``FillFunctor<long>``) in the trace
just before its replays, so the trace splits into one segment per workload at
those blocks.  For each workload the summary gives its roofline kernel's
launches in that segment, the mean duration (End - Start) of the last
``steps`` of them -- the timed replay -- and bench.py's hipEvent time per step
from the JSON line; then the run's per-kernel statistics (rocprofv3's
``kernel_stats.csv``).
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import sys

from tilebench_amd.profiling.kernels import demangle, kernel_stem

_FILL = "FillFunctor<long>"


def _one(path: str, pattern: str) -> str:
    hits = sorted(glob.glob(os.path.join(path, "**", pattern), recursive=True))
    if not hits:
        raise FileNotFoundError(f"no {pattern} under {path}")
    return hits[0]


def bench_line(path: str) -> dict:
    """The JSON line bench.py printed (the last line of the file that starts with '{')."""
    with open(path) as f:
        lines = [ln for ln in f if ln.startswith("{")]
    if not lines:
        raise ValueError(f"no bench.py JSON line in {path}")
    return json.loads(lines[-1])


def workloads(line: dict) -> list[tuple[str, str, float]]:
    """[(workload, roofline kernel, ms per step)] in the order bench.py ran them."""
    out = [(line["config"]["workload"] + " (headline)", line["roofline"]["kernel"], line["ms_per_step"])]
    for name, r in (line.get("suite") or {}).items():
        out.append((name, r["kernel"], r["ms"]))
    return out


def launches(trace_csv: str) -> list[tuple[str, int, int]]:
    with open(trace_csv, newline="") as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    return [(kernel_stem(demangle(r["Kernel_Name"])), int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
            for r in rows]


def segments(recs, n: int) -> list[tuple[int, int]]:
    """[lo, hi) index ranges of the n workload segments (each starts at a fill block)."""
    starts = [i for i, r in enumerate(recs) if _FILL in r[0] and (i == 0 or _FILL not in recs[i - 1][0])]
    if len(starts) != n:
        raise ValueError(f"{len(starts)} fill blocks in the trace for {n} workloads")
    return [(lo, starts[j + 1] if j + 1 < n else len(recs)) for j, lo in enumerate(starts)]


def summarize(trace_dir: str, bench_json: str) -> str:
    line = bench_line(bench_json)
    steps = int(line["steps"])
    wl = workloads(line)
    recs = launches(_one(trace_dir, "*kernel_trace.csv"))
    out = [f"{'workload':28s} {'kernel':40s} {'launches':>8s} {'timed_avg_us':>12s} {'bench_us/step':>13s}"]
    for (name, kernel, ms), (lo, hi) in zip(wl, segments(recs, len(wl))):
        idx = [i for i in range(lo, hi) if recs[i][0] == kernel]
        timed = idx[-steps:]
        avg = sum(recs[i][2] - recs[i][1] for i in timed) / max(len(timed), 1) / 1e3
        out.append(f"{name:28s} {kernel[:40]:40s} {len(idx):8d} {avg:12.2f} {ms * 1e3:13.2f}")
    out += ["", "All kernels of the run (kernel_stats.csv), microseconds:", "",
            f"{'kernel':60s} {'calls':>7s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s}"]
    with open(_one(trace_dir, "*kernel_stats.csv"), newline="") as f:
        for r in csv.DictReader(f):
            name = kernel_stem(demangle(r["Name"]))
            out.append(f"{name[:60]:60s} {int(r['Calls']):7d} {float(r['AverageNs']) / 1e3:9.2f} "
                       f"{float(r['MinNs']) / 1e3:9.2f} {float(r['MaxNs']) / 1e3:9.2f}")
    return "\n".join(out)


def timeline(trace_dir: str, kernel_regex: str = "") -> str:
    recs = launches(_one(trace_dir, "*kernel_trace.csv"))
    pat = re.compile(kernel_regex)
    picked = [i for i, r in enumerate(recs) if r[0].startswith("tb::") and pat.search(r[0])]
    if not picked:
        return "no matching launch"
    t0 = recs[picked[0]][1]
    out = [f"{'kernel':44s} {'start_us':>11s} {'dur_us':>9s}  {'gap_us':>8s} previous kernel"]
    for i in picked:
        name, s, e = recs[i]
        prev = f"{(s - recs[i - 1][2]) / 1e3:8.2f} {recs[i - 1][0][:44]}" if i else ""
        out.append(f"{name[:44]:44s} {(s - t0) / 1e3:11.1f} {(e - s) / 1e3:9.2f}  {prev}")
    return "\n".join(out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("suite", help="per-workload durations of a bench.py trace")
    s.add_argument("trace_dir", help="rocprofv3 output directory (kernel_trace.csv, kernel_stats.csv)")
    s.add_argument("bench_json", help="file holding bench.py's JSON line from the same run")
    t = sub.add_parser("launches", help="the backend's launches in trace order")
    t.add_argument("trace_dir")
    t.add_argument("--kernel", default="", help="regex on the kernel name")
    args = ap.parse_args(argv)
    print(summarize(args.trace_dir, args.bench_json) if args.cmd == "suite" else
          timeline(args.trace_dir, args.kernel))
    return 0


if __name__ == "__main__":
    sys.exit(main())
