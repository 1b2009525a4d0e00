"""Derived performance metrics (tilebench/core/metrics.py:57-121) and the
roofline fraction (tilebench/llm/roofline.py:41-109)."""
from __future__ import annotations

import json
import math
import os

from tilebench_amd.backends import BACKEND_ORDER
from tilebench_amd.core.dtypes import dtype_size
from tilebench_amd.paths import PEAK_PERFORMANCE_ROOT

BACKENDS = ("torch",) + BACKEND_ORDER
NON_GPU_BACKENDS = ("nki",)


def load_peak_config(gpu_name: str) -> dict:
    """Peaks of `gpu_name`: data/peak_performance/<gpu>.json if present, else the
    calibrated file data/peak_performance/empirical/<gpu>.json (MI355X has only
    the calibrated one: tilebench_amd.calibration writes it), else {}."""
    for path in (os.path.join(PEAK_PERFORMANCE_ROOT, f"{gpu_name}.json"),
                 os.path.join(PEAK_PERFORMANCE_ROOT, "empirical", f"{gpu_name}.json")):
        if os.path.isfile(path):
            with open(path) as f:
                return json.load(f)
    return {}


def _eval_expr(expr, ctx: dict):
    if not expr:
        return None
    try:
        return float(eval(str(expr), {"__builtins__": {}, "math": math}, ctx))  # noqa: S307 (package configs)
    except Exception:
        return None


def eval_ctx(params: dict, dtype_str: str, problem_size: int | None = None) -> dict:
    ctx = {"n": int(params.get("n", problem_size or 1)), "dtype_size": dtype_size(dtype_str)}
    ctx.update({k: v for k, v in params.items() if isinstance(v, (int, float))})
    return ctx


def work(metrics_cfg: dict, params: dict, dtype_str: str) -> tuple[float | None, float | None]:
    """(flops, bytes) of one call from the config's flops_expr / bytes_expr."""
    ctx = eval_ctx(params, dtype_str)
    return _eval_expr(metrics_cfg.get("flops_expr"), ctx), _eval_expr(metrics_cfg.get("bytes_expr"), ctx)


def applicable_backends(peak_cfg: dict | None) -> tuple[str, ...]:
    declared = (peak_cfg or {}).get("backends")
    if declared:
        return tuple(declared)
    return tuple(b for b in BACKENDS if b not in NON_GPU_BACKENDS)


def compute_derived(result: dict, metrics_cfg: dict, peak_cfg: dict | None = None) -> dict:
    """Per-backend latency, GB/s, TFLOPS, %peak, AI and speedup over torch."""
    params = result.get("params", {})
    flops, nbytes = work(metrics_cfg, params, result.get("dtype", "fp32"))
    peak = peak_cfg or {}
    peak_bw = peak.get("peak_bw_GBs") or metrics_cfg.get("peak_bw_GBs")
    peak_bw = float(peak_bw) if peak_bw is not None else None
    peak_mode = metrics_cfg.get("peak_tflops_key") or result.get("dtype")
    table = {**(peak.get("peak_tops") or {}), **(peak.get("peak_tflops") or {})}
    # a case dtype names its matrix peak with the calibration's "_mma" suffix
    raw = table.get(peak_mode, table.get(f"{peak_mode}_mma"))
    peak_tf = float(raw) if raw is not None else None
    torch_ms = result.get("torch_ms")
    torch_ms = float(torch_ms) if torch_ms is not None and torch_ms > 0 and not math.isnan(torch_ms) else None
    out = {}
    for backend in BACKENDS:
        ms = result.get(f"{backend}_ms")
        if ms is None or not (float(ms) > 0):
            continue
        ms = float(ms)
        d = {"latency_ms": ms}
        applies = backend in applicable_backends(peak)
        if nbytes:
            d["bandwidth_GBs"] = nbytes / (ms * 1e-3) / 1e9
            if applies and peak_bw:
                d["pct_peak_bw"] = d["bandwidth_GBs"] / peak_bw * 100.0
        if flops:
            d["tflops"] = flops / (ms * 1e-3) / 1e12
            if applies and peak_tf:
                d["pct_peak_tflops"] = d["tflops"] / peak_tf * 100.0
        if flops and nbytes:
            d["arithmetic_intensity"] = flops / nbytes
        if backend != "torch" and torch_ms is not None:
            d["speedup"] = torch_ms / ms
        out[backend] = d
    return out


def roofline_pct(flops: float, nbytes: float, latency_s: float, peak_bw_GBs: float,
                 peak_tflops: float | None, bound: str | None = None) -> dict:
    """Fraction of the roofline ceiling min(P, BW * AI) reached.

    bound="hbm" treats the kernel as pure data movement (measured GB/s over the
    bandwidth peak), bound="mfma" as compute (measured TFLOPS over P), None
    picks the lower ceiling as the reference does."""
    if latency_s <= 0:
        raise ValueError("non-positive latency")
    bw = nbytes / latency_s
    perf = flops / latency_s if flops else 0.0
    peak_bw = peak_bw_GBs * 1e9
    if bound == "hbm" or not flops:
        return {"bound_by": "hbm", "achieved": bw / 1e9, "peak": peak_bw_GBs, "unit": "GB/s",
                "frac": bw / peak_bw}
    if bound == "mfma":
        return {"bound_by": "mfma", "achieved": perf / 1e12, "peak": peak_tflops, "unit": "TFLOP/s",
                "frac": perf / (peak_tflops * 1e12)}
    ceiling = min(peak_tflops * 1e12, peak_bw * flops / nbytes) if peak_tflops else peak_bw * flops / nbytes
    return {"bound_by": "mfma" if peak_tflops and peak_tflops * 1e12 < peak_bw * flops / nbytes else "hbm",
            "achieved": perf / 1e12, "peak": ceiling / 1e12, "unit": "TFLOP/s", "frac": perf / ceiling}
