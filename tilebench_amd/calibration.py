"""Empirical peaks of the GPU this process runs on, measured by a fixed protocol.

The reference calibrates its roofline ceilings this way
(tilebench/llm/v2/calibration/protocol.py:10-34, stats.py:39-60,
gpu_probes.py:225, 284) and stores the result per GPU
(tilebench/data/peak_performance/empirical/MI300X.json).  This module does the
same for MI355X with this package's probes and torch's library GEMMs, and
writes the same keys (``peak_bw_GBs``, ``peak_tflops.{fp16,bf16,fp8_e4m3fn}_mma``,
``peak_tops.int8_mma``) plus every point it measured.

Protocol (``PROTOCOL``):
  * a point is a launchable callable; after `warmup` launches, the number of
    launches per sample is raised until one sample takes `target_sample_ms`;
    then `batches` batches of `repeat` samples, each timed with hipEvents
    around back-to-back launches; point time = the median over batches of each
    batch's median (never the fastest sample);
  * HBM: the library's copy probe and torch's device copy, over sizes whose
    working set (read + written) is at least 4x the last-level cache are
    eligible; the peak is the largest eligible throughput, and the eligible
    points of the probe that gives it must agree within 5 % (a plateau);
    smaller sizes are kept as cache-scale diagnostics;
  * matrix: per operand type, the library GEMM (torch.matmul, torch._scaled_mm,
    torch._int_mm) at square sizes, each checked on a block against float64
    (integer: exactly), and the instruction-level probe tb_probe_mfma (8
    independent 32x32 MFMA chains per wavefront) at 1, 2 and 4 blocks per CU;
    the peak is the largest valid throughput.  Including the probe makes the
    peak the matrix pipe's own ceiling, not only what a library GEMM reaches.

Usage (on the GPU):
    python -m tilebench_amd.calibration --out tilebench_amd/data/peak_performance/empirical/MI355X.json
"""
from __future__ import annotations

import argparse
import hashlib
import json
import math
import statistics
import sys
import time

MIB = 1024 * 1024

PROTOCOL = {
    "protocol": "tbhip-empirical-roofline/1",
    "follows": "tilebench-empirical-roofline/2 (tilebench/llm/v2/calibration/protocol.py)",
    "batches": 3,
    "warmup": 10,
    "repeat": 15,
    "target_sample_ms": 2.0,
    "statistic": "per point: median of each batch's samples, then the median of the batch medians; "
                 "peak: the largest throughput over the valid points (HBM: eligible points on a plateau)",
    "batch_spread_flag": 0.03,
    "hbm": {"probes": ["tb_probe_copy", "torch_copy"], "sizes_mib": [16, 64, 256, 512, 1024, 2048],
            "min_working_set_over_llc": 4.0, "plateau_tolerance": 0.05},
    "mma": {"gemm_sizes": [4096, 8192, 16384], "check_block": 128, "probe_blocks_per_cu": [1, 2, 4],
            "probe_iters": 2000},
}

# ----------------------------------------------------------------------------- statistics


def summarize_batches(batches: list[list[float]]) -> dict:
    """The protocol's reading of one point's samples: the median of each batch,
    the point time (the median of those medians, so that no single sample,
    fastest or slowest, sets it) and the batches' relative spread (range of
    the batch medians over the point time)."""
    if len(batches) == 0:
        raise ValueError("a point needs at least one batch of samples")
    per_batch = []
    for i, samples in enumerate(batches):
        if len(samples) == 0:
            raise ValueError(f"batch {i} of the point holds no samples")
        per_batch.append(statistics.median(samples))
    mid = statistics.median(per_batch)
    return {"medians": per_batch, "time": mid, "spread": (max(per_batch) - min(per_batch)) / mid}


def point_time(batches: list[list[float]]) -> float:
    return summarize_batches(batches)["time"]


def hbm_eligible(working_set: int, llc: int | None, factor: float) -> bool:
    """A point measures HBM only if its working set is at least `factor` x the
    last-level cache; with the cache size unknown no point qualifies."""
    if llc is None or llc <= 0:
        return False
    return working_set >= factor * llc


def select_peak(points: list[dict], bandwidth: bool, plateau_tolerance: float = 0.05) -> dict:
    """The calibrated value of one mode from its points (dicts with
    `throughput`, `valid`, and for bandwidth `eligible`, `probe`)."""
    pool = [p for p in points if p.get("valid") and (p.get("eligible") if bandwidth else True)]
    if not pool:
        return {"status": "failed", "value": None, "selected": None, "reason": "no valid point"}
    best = max(pool, key=lambda p: p["throughput"])
    res = {"status": "calibrated", "value": best["throughput"], "selected": best["id"], "reason": None}
    if bandwidth:
        same = [p["throughput"] for p in pool if p["probe"] == best["probe"]]
        spread = (max(same) - min(same)) / max(same) if len(same) > 1 else None
        res["plateau"] = {"probe": best["probe"], "points": len(same), "spread": spread}
        if spread is None or spread > plateau_tolerance:
            res.update(status="failed", value=None,
                       reason=f"{best['probe']} shows no plateau over HBM-scale sizes (spread {spread})")
    return res


# ----------------------------------------------------------------------------- timing


def measure(fn, proto: dict) -> dict:
    """Per-launch milliseconds of fn in `batches` x `repeat` samples."""
    import torch

    for _ in range(proto["warmup"]):
        fn()
    torch.cuda.synchronize()
    inner = 1
    while True:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(inner):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
        if ms >= proto["target_sample_ms"] or inner >= 4096:
            break
        inner = min(4096, max(inner * 2, int(inner * proto["target_sample_ms"] / max(ms, 1e-3)) + 1))
    batches = []
    for _ in range(proto["batches"]):
        starts = [torch.cuda.Event(enable_timing=True) for _ in range(proto["repeat"])]
        stops = [torch.cuda.Event(enable_timing=True) for _ in range(proto["repeat"])]
        for a, b in zip(starts, stops):
            a.record()
            for _ in range(inner):
                fn()
            b.record()
        torch.cuda.synchronize()
        batches.append([a.elapsed_time(b) / inner for a, b in zip(starts, stops)])
    return {"inner": inner, "batches_ms": batches}


def _point(pid: str, work: float, meas: dict, valid: bool, **extra) -> dict:
    summ = summarize_batches(meas["batches_ms"])
    t = summ["time"] / 1e3
    return {"id": pid, "work": work, "inner": meas["inner"], "batch_medians_ms": summ["medians"],
            "point_time_s": t, "throughput": work / t, "batch_spread": summ["spread"],
            "valid": bool(valid), **extra}


# ----------------------------------------------------------------------------- probes


def hbm_points(proto: dict, llc: int | None) -> list[dict]:
    import torch

    from tilebench_amd import runtime as rt

    stream = rt.stream_handle()
    pts = []
    for probe in proto["hbm"]["probes"]:
        for size in proto["hbm"]["sizes_mib"]:
            n = size * MIB
            g = torch.Generator(device="cuda").manual_seed(77 + size)
            src = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda", generator=g)
            dst = torch.empty_like(src)
            if probe == "tb_probe_copy":
                fn = (lambda s=src, d=dst, n=n: rt.call("tb_probe_copy", s.data_ptr(), d.data_ptr(), n, stream))
            else:
                fn = (lambda s=src, d=dst: d.copy_(s))
            fn()
            torch.cuda.synchronize()
            ok = bool(torch.equal(dst, src))
            meas = measure(fn, proto)
            ws = 2 * n
            pts.append(_point(f"{probe}/{size}MiB", 2.0 * n, meas, ok, probe=probe, size_mib=size,
                              working_set_bytes=ws,
                              eligible=hbm_eligible(ws, llc, proto["hbm"]["min_working_set_over_llc"]),
                              check={"ok": ok, "rule": "dst equals src (random bytes)"}))
            del src, dst
            torch.cuda.empty_cache()
    for p in pts:
        p["throughput_GBs"] = p["throughput"] / 1e9
    return pts


_GEMM = {  # mode -> (torch dtype name, api, rel-RMS window against float64)
    "fp16_mma": ("float16", "matmul", 1e-2),
    "bf16_mma": ("bfloat16", "matmul", 2e-2),
    "fp8_e4m3fn_mma": ("float8_e4m3fn", "_scaled_mm", 2e-2),
    "int8_mma": ("int8", "_int_mm", 0.0),
}
_PROBE_KIND = {"fp16_mma": (0, 32768), "fp8_e4m3fn_mma": (1, 131072), "bf16_mma": (2, 32768), "int8_mma": (3, 65536)}


def gemm_points(mode: str, proto: dict) -> list[dict]:
    import torch

    dname, api, window = _GEMM[mode]
    dt = getattr(torch, dname)
    pts = []
    blk = proto["mma"]["check_block"]
    for m in proto["mma"]["gemm_sizes"]:
        pid = f"{mode}/{api}/M{m}"
        g = torch.Generator(device="cuda").manual_seed(1000 + m)
        try:
            if api == "_int_mm":
                a = torch.randint(-8, 8, (m, m), dtype=torch.int8, device="cuda", generator=g)
                b = torch.randint(-8, 8, (m, m), dtype=torch.int8, device="cuda", generator=g)
                fn = (lambda a=a, b=b: torch._int_mm(a, b))
            elif api == "_scaled_mm":
                a = torch.randn(m, m, device="cuda", generator=g).to(dt)
                b = torch.randn(m, m, device="cuda", generator=g).to(dt).t()  # column-major operand
                one = torch.ones((), device="cuda", dtype=torch.float32)
                fn = (lambda a=a, b=b, one=one: torch._scaled_mm(a, b, scale_a=one, scale_b=one,
                                                                 out_dtype=torch.bfloat16))
            else:
                a = torch.randn(m, m, device="cuda", generator=g).to(dt)
                b = torch.randn(m, m, device="cuda", generator=g).to(dt)
                fn = (lambda a=a, b=b: torch.matmul(a, b))
            c = fn()
            torch.cuda.synchronize()
            if api == "_int_mm":
                ref = a[:blk].cpu().long() @ b[:, :blk].cpu().long()
                ok = bool(torch.equal(c[:blk, :blk].cpu().long(), ref))
                check = {"ok": ok, "rule": "int64 CPU product of a block, exact"}
            else:
                ref = a[:blk].double() @ b[:, :blk].double()
                got = c[:blk, :blk].double()
                rel = float(torch.sqrt(((got - ref) ** 2).mean()) / torch.sqrt((ref ** 2).mean()))
                ok = math.isfinite(rel) and rel < window
                check = {"ok": ok, "rel_rms_error": rel, "max": window, "rule": "block rel-RMS vs float64"}
            del c
            meas = measure(fn, proto)
            pts.append(_point(pid, 2.0 * m ** 3, meas, ok, source="library GEMM (torch." + api + ")", M=m, check=check))
        except (RuntimeError, TypeError, ValueError) as e:
            pts.append({"id": pid, "valid": False, "error": f"{type(e).__name__}: {e}"})
        torch.cuda.empty_cache()
    return pts


def probe_points(mode: str, proto: dict) -> list[dict]:
    import torch

    from tilebench_amd import runtime as rt

    kind, per_mfma = _PROBE_KIND[mode]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    iters = proto["mma"]["probe_iters"]
    stream = rt.stream_handle()
    pts = []
    for bpc in proto["mma"]["probe_blocks_per_cu"]:
        blocks = bpc * cus
        out = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
        fn = (lambda out=out, blocks=blocks: rt.call("tb_probe_mfma", kind, blocks, iters, out.data_ptr(), stream))
        fn()
        torch.cuda.synchronize()
        ok = bool(torch.isfinite(out).all())
        meas = measure(fn, proto)
        work = float(blocks * 4 * 8 * iters * per_mfma)
        pts.append(_point(f"{mode}/tb_probe_mfma/{bpc}_per_cu", work, meas, ok, source="instruction probe",
                          blocks_per_cu=bpc, check={"ok": ok, "rule": "outputs finite"}))
    return pts


# ----------------------------------------------------------------------------- run


def environment() -> dict:
    import platform

    import torch

    props = torch.cuda.get_device_properties(0)
    return {"gpu": props.name, "gcn_arch": getattr(props, "gcnArchName", None), "cus": props.multi_processor_count,
            "torch": torch.__version__, "hip": torch.version.hip, "host": platform.node(),
            "utc": time.strftime("%Y%m%dT%H%M%SZ", time.gmtime())}


def gpu_model(env: dict) -> str:
    """Model name for the peak file.  The runtime's marketing name is missing
    when the host lacks the amdgpu.ids table ("AMD Radeon Graphics"); a
    gfx950 device with 256 CUs is then taken to be the MI355X this package
    targets (the MI350X shares the die and CU count at a lower power limit)."""
    for tag in ("MI355X", "MI350X", "MI325X", "MI300X"):
        if tag in env["gpu"]:
            return tag
    if (env.get("gcn_arch") or "").startswith("gfx950") and env.get("cus") == 256:
        return "MI355X"
    return env["gpu"].replace(" ", "_")


def calibrate(proto: dict = PROTOCOL, modes=tuple(_GEMM)) -> dict:
    from tilebench_amd import hardware
    from tilebench_amd import runtime as rt

    rt.require_device()
    rt.load_library()
    env = environment()
    llc = hardware.last_level_cache_bytes()
    hbm = hbm_points(proto, llc)
    bw = select_peak(hbm, bandwidth=True, plateau_tolerance=proto["hbm"]["plateau_tolerance"])
    modes_out = {"hbm": {"selection": bw, "points": hbm}}
    tflops, tops = {}, {}
    for mode in modes:
        pts = gemm_points(mode, proto) + probe_points(mode, proto)
        sel = select_peak(pts, bandwidth=False)
        modes_out[mode] = {"selection": sel, "points": pts}
        lib = [p["throughput"] for p in pts if p.get("valid") and p.get("source", "").startswith("library")]
        sel["library_gemm_best"] = max(lib) / 1e12 if lib else None
        if sel["value"] is not None:
            (tops if mode == "int8_mma" else tflops)[mode] = round(sel["value"] / 1e12, 2)
    proto_hash = hashlib.sha256(json.dumps(proto, sort_keys=True).encode()).hexdigest()[:8]
    name = gpu_model(env)
    return {
        "gpu": f"AMD Instinct {name}",
        "peak_bw_GBs": round(bw["value"] / 1e9, 2) if bw["value"] else None,
        "peak_tflops": tflops,
        "peak_tops": tops,
        "calibration_id": f"{name}-{env['utc']}-{proto_hash}",
        "environment": env,
        "last_level_cache_bytes": llc,
        "protocol": proto,
        "modes": modes_out,
    }


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--out", default=None, help="write the calibration JSON here")
    args = ap.parse_args(argv)
    res = calibrate()
    summary = {k: res[k] for k in ("gpu", "peak_bw_GBs", "peak_tflops", "peak_tops", "calibration_id")}
    print(json.dumps(summary), flush=True)
    for mode, m in res["modes"].items():
        for p in m["points"]:
            if "throughput" in p:
                unit = 1e9 if mode == "hbm" else 1e12
                print(f"  {p['id']:40s} {p['throughput'] / unit:10.2f} {'GB/s' if mode == 'hbm' else 'T/s'}"
                      f"  valid={p['valid']}  spread={p['batch_spread']:.3f}", flush=True)
            else:
                print(f"  {p['id']:40s} invalid: {p.get('error')}", flush=True)
    if args.out:
        with open(args.out, "w") as f:
            json.dump(res, f, indent=1)
            f.write("\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
