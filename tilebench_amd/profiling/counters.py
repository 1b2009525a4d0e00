"""Summaries of rocprofv3 counter captures of the hip backend.

Reads the ``*counter_collection.csv`` files that ``rocprofv3 --pmc ... --output-format csv``
writes and reduces them to per-dispatch means per kernel (every counter value
of a dispatch is summed over the GPU, as rocprofv3 reports it).

    python -m tilebench_amd.profiling.counters summary DIR [DIR ...] [--kernel REGEX]
        one block per kernel: each counter's mean per dispatch, and the derived
        ratios (MFMA utilisation, wait fractions, VALU instructions per MFMA)

    python -m tilebench_amd.profiling.counters traffic FETCH_DIR WRITE_DIR [--out traffic.json]
        HBM bytes per launch of every kernel from a FETCH_SIZE and a WRITE_SIZE
        pass (KiB per dispatch), each scaled by what the counter reads for the
        copy probe (tb::copy_kernel, 16 bytes per thread each way) in the same pass; merged
        into an existing traffic.json (kernels not in these passes are kept)

    python -m tilebench_amd.profiling.counters table FETCH_DIR WRITE_DIR BENCH_JSON
        the same scaled bytes per workload of a bench.py run (BENCH_JSON: the
        JSON line that pass printed), beside the workload's algorithmic reads
        and writes: each workload's roofline kernel, averaged over its own
        dispatches (the run splits into workloads at the fill launches that
        graph capture leaves before each workload's replays)

Derived ratios: MFMA utilisation = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8
XCDs x 1024 SIMDs); SQ cycle counters are in units of four cycles per wave.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import sys
from collections import defaultdict

from tilebench_amd.profiling.kernels import kernel_stem

COPY_KERNEL = "tb::copy_kernel"
XCDS, SIMDS = 8, 1024


def counter_files(path: str) -> list[str]:
    if os.path.isfile(path):
        return [path]
    return sorted(glob.glob(os.path.join(path, "**", "*counter_collection.csv"), recursive=True))


def per_dispatch(paths, kernel_regex: str | None = None) -> dict:
    """{kernel stem: {"dispatches": n, "counters": {name: mean per dispatch}}}."""
    pat = re.compile(kernel_regex) if kernel_regex else None
    sums: dict = defaultdict(lambda: defaultdict(float))
    seen: dict = defaultdict(lambda: defaultdict(set))   # kernel -> counter -> dispatches reporting it
    for path in paths:
        for f in counter_files(path):
            with open(f, newline="") as fh:
                for r in csv.DictReader(fh):
                    name = kernel_stem(r["Kernel_Name"])
                    if pat and not pat.search(name):
                        continue
                    sums[name][r["Counter_Name"]] += float(r["Counter_Value"])
                    seen[name][r["Counter_Name"]].add((f, r["Dispatch_Id"]))
    out = {}
    for name, cs in sums.items():
        counts = {k: len(v) for k, v in seen[name].items()}
        out[name] = {"dispatches": max(counts.values()),
                     "counters": {k: v / counts[k] for k, v in sorted(cs.items())}}
    return out


def derived(c: dict) -> dict:
    """Ratios of one kernel's per-dispatch counters (those whose inputs are present)."""
    d = {}
    g = c.get("GRBM_GUI_ACTIVE")
    if g and "SQ_VALU_MFMA_BUSY_CYCLES" in c:
        d["mfma_utilisation"] = c["SQ_VALU_MFMA_BUSY_CYCLES"] / (g / XCDS * SIMDS)
    w = c.get("SQ_WAVE_CYCLES")
    if w:
        for k in ("SQ_WAIT_INST_ANY", "SQ_WAIT_ANY", "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS"):
            if k in c:
                d[k.lower() + "_per_wave_cycle"] = c[k] / w
    if c.get("SQ_INSTS_MFMA"):
        if "SQ_INSTS_VALU" in c:
            d["valu_per_mfma"] = c["SQ_INSTS_VALU"] / c["SQ_INSTS_MFMA"]
        if "SQ_VALU_MFMA_BUSY_CYCLES" in c:
            d["mfma_busy_cycles_per_instruction"] = c["SQ_VALU_MFMA_BUSY_CYCLES"] / c["SQ_INSTS_MFMA"]
    if c.get("SQ_WAVES") and "SQ_INSTS_VALU" in c:
        d["valu_per_wave"] = c["SQ_INSTS_VALU"] / c["SQ_WAVES"]
    return d


def format_summary(res: dict) -> str:
    lines = []
    for name, r in sorted(res.items()):
        lines.append(f"## {name}, {r['dispatches']} dispatches")
        for k, v in r["counters"].items():
            lines.append(f"  {k:40s} {v:20,.0f}")
        for k, v in derived(r["counters"]).items():
            lines.append(f"  -> {k} {v:.4g}")
        lines.append("")
    return "\n".join(lines)


def copy_factor(path: str, counter: str) -> float:
    """Known bytes / counted bytes over the copy probe's dispatches in one pass.
    The probe copies 16 bytes per thread each way (tb_probe_copy), so a
    dispatch's bytes are its grid size x 16 whatever size the run used (the
    bench's own copy line moves 512 MiB, its live peak measurement 1 GiB)."""
    ratios = []
    for f in counter_files(path):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                if kernel_stem(r["Kernel_Name"]) == COPY_KERNEL and r["Counter_Name"] == counter:
                    ratios.append(int(r["Grid_Size"]) * 16 / (float(r["Counter_Value"]) * 1024))
    if not ratios:
        raise ValueError(f"no copy-probe dispatch in {path}: run the pass with bench.py's hbm_copy_probe")
    ratios.sort()
    return ratios[len(ratios) // 2]


def traffic(fetch_dir: str, write_dir: str) -> dict:
    """{kernel: {"fetch_bytes", "write_bytes", "fetch_factor", "write_factor"}} of the
    backend's kernels (tb::): KiB per dispatch x 1024, scaled so that the copy probe
    reads its known bytes.  The probe itself is left out (its dispatches move 512 MiB
    or 1 GiB, so a mean over them describes neither)."""
    fetch = per_dispatch([fetch_dir])
    write = per_dispatch([write_dir])
    ff, wf = copy_factor(fetch_dir, "FETCH_SIZE"), copy_factor(write_dir, "WRITE_SIZE")
    out = {}
    for name in sorted(set(fetch) & set(write)):
        if name == COPY_KERNEL or not name.startswith("tb::"):
            continue
        out[name] = {"fetch_bytes": int(round(fetch[name]["counters"]["FETCH_SIZE"] * 1024 * ff)),
                     "write_bytes": int(round(write[name]["counters"]["WRITE_SIZE"] * 1024 * wf)),
                     "fetch_factor": round(ff, 4), "write_factor": round(wf, 4)}
    return out


def _dispatches(path: str, counter: str) -> list[tuple[str, float]]:
    """[(kernel stem, counter value)] of one pass in dispatch order."""
    rows = []
    for f in counter_files(path):
        with open(f, newline="") as fh:
            rows += [(int(r["Dispatch_Id"]), kernel_stem(r["Kernel_Name"]), float(r["Counter_Value"]))
                     for r in csv.DictReader(fh) if r["Counter_Name"] == counter]
    rows.sort()
    return [(k, v) for _, k, v in rows]


def workload_table(fetch_dir: str, write_dir: str, bench_json: str) -> list[dict]:
    """Per workload of the bench run: its roofline kernel's scaled FETCH/WRITE bytes per
    launch (mean over the workload's own dispatches of it) and its algorithmic bytes."""
    from tilebench_amd.profiling.suite_trace import bench_line, segments, workloads

    line = bench_line(bench_json)
    wl = workloads(line)
    alg = {wl[0][0]: line["roofline"]}
    alg.update(line.get("suite") or {})
    out = []
    per_pass = {}
    for d, counter in ((fetch_dir, "FETCH_SIZE"), (write_dir, "WRITE_SIZE")):
        recs = _dispatches(d, counter)
        per_pass[counter] = (recs, segments(recs, len(wl)), copy_factor(d, counter))
    for j, (name, kernel, _) in enumerate(wl):
        row = {"workload": name, "kernel": kernel,
               "alg_read_bytes": alg[name].get("alg_read_bytes"), "alg_write_bytes": alg[name].get("alg_write_bytes")}
        for counter, key in (("FETCH_SIZE", "fetch_bytes"), ("WRITE_SIZE", "write_bytes")):
            recs, segs, factor = per_pass[counter]
            lo, hi = segs[j]
            vals = [v for k, v in recs[lo:hi] if k == kernel]
            row[key] = sum(vals) / len(vals) * 1024 * factor if vals else None
            row["dispatches"] = len(vals)
        out.append(row)
    return out


def format_table(rows: list[dict]) -> str:
    def kib(v):
        return "-" if v is None else f"{v / 1024:.0f}"

    def ratio(a, b):
        return "-" if a is None or not b else f"{a / b:.2f}"

    lines = [f"{'workload':28s} {'kernel':42s} {'fetch_KiB':>10s} {'alg_rd_KiB':>10s} {'x':>6s} "
             f"{'write_KiB':>10s} {'alg_wr_KiB':>10s} {'x':>6s}"]
    for r in rows:
        lines.append(f"{r['workload'][:28]:28s} {r['kernel'][:42]:42s} {kib(r['fetch_bytes']):>10s} "
                     f"{kib(r['alg_read_bytes']):>10s} {ratio(r['fetch_bytes'], r['alg_read_bytes']):>6s} "
                     f"{kib(r['write_bytes']):>10s} {kib(r['alg_write_bytes']):>10s} "
                     f"{ratio(r['write_bytes'], r['alg_write_bytes']):>6s}")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("summary")
    s.add_argument("dirs", nargs="+")
    s.add_argument("--kernel", default=None, help="regex on the kernel name")
    t = sub.add_parser("traffic")
    t.add_argument("fetch_dir")
    t.add_argument("write_dir")
    t.add_argument("--out", default=None, help="traffic.json to update (printed when omitted)")
    t.add_argument("--workload", default="", help="text stored with each updated kernel")
    b = sub.add_parser("table")
    b.add_argument("fetch_dir")
    b.add_argument("write_dir")
    b.add_argument("bench_json", help="bench.py's JSON line from one of the two passes")
    args = ap.parse_args(argv)
    if args.cmd == "summary":
        print(format_summary(per_dispatch(args.dirs, args.kernel)))
        return 0
    if args.cmd == "table":
        print(format_table(workload_table(args.fetch_dir, args.write_dir, args.bench_json)))
        return 0
    new = traffic(args.fetch_dir, args.write_dir)
    if args.out is None:
        print(json.dumps(new, indent=1))
        return 0
    doc = {"note": "HBM traffic per launch (bytes), FETCH_SIZE/WRITE_SIZE scaled by the copy-probe factors",
           "kernels": {}}
    if os.path.exists(args.out):
        with open(args.out) as f:
            doc = json.load(f)
    for name, v in new.items():
        if args.workload:
            v["workload"] = args.workload
        doc["kernels"][name] = v
    with open(args.out, "w") as f:
        json.dump(doc, f, indent=1)
    print(f"updated {len(new)} kernels in {args.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
