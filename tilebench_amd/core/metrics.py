"""Derived performance metrics of one case (tilebench/core/metrics.py:57-121:
GB/s, TFLOPS, % of peak, arithmetic intensity, speedup over torch) and the
roofline fraction (tilebench/llm/roofline.py:41-109).

Peaks come in two files, as in the reference's data/peak_performance/:
``<gpu>.json`` holds the published (datasheet) figures and is what ``pct_peak_*``
divides by, as the reference's core metrics do; ``empirical/<gpu>.json`` holds
the peaks measured on the box by tilebench_amd.calibration, and when it is
given ``compute_derived`` also reports ``pct_calibrated_peak_*`` against it.
"""
from __future__ import annotations

import ast
import json
import math
import operator
import os

from tilebench_amd.backends import BACKEND_ORDER
from tilebench_amd.core.dtypes import dtype_size
from tilebench_amd.paths import PEAK_PERFORMANCE_ROOT

BACKENDS = ("torch",) + BACKEND_ORDER
#: backends that do not run on the GPU a peak file describes (no % of peak for them)
NON_GPU_BACKENDS = ("nki",)


def _read_json(path: str) -> dict:
    if not os.path.isfile(path):
        return {}
    with open(path) as f:
        return json.load(f)


def load_peak_config(gpu_name: str) -> dict:
    """Published peaks of `gpu_name` (data/peak_performance/<gpu>.json), or {}."""
    return _read_json(os.path.join(PEAK_PERFORMANCE_ROOT, f"{gpu_name}.json"))


def load_calibrated_peaks(gpu_name: str) -> dict:
    """Peaks measured on the box (data/peak_performance/empirical/<gpu>.json,
    written by `python -m tilebench_amd.calibration`), or {}."""
    return _read_json(os.path.join(PEAK_PERFORMANCE_ROOT, "empirical", f"{gpu_name}.json"))


# ----------------------------------------------------------------------------- config expressions

_BINARY = {ast.Add: operator.add, ast.Sub: operator.sub, ast.Mult: operator.mul, ast.Div: operator.truediv,
           ast.FloorDiv: operator.floordiv, ast.Mod: operator.mod, ast.Pow: operator.pow}
_UNARY = {ast.USub: operator.neg, ast.UAdd: operator.pos}
_CALLS = {"min": min, "max": max, "abs": abs, "int": int, "float": float,
          "ceil": math.ceil, "floor": math.floor, "log2": math.log2, "sqrt": math.sqrt}


def _walk(node, ctx: dict):
    """Value of an arithmetic expression tree: numbers, names bound in `ctx`,
    + - * / // % **, unary signs and a few pure functions (also as math.f)."""
    if isinstance(node, ast.Expression):
        return _walk(node.body, ctx)
    if isinstance(node, ast.Constant) and isinstance(node.value, (int, float)) and not isinstance(node.value, bool):
        return node.value
    if isinstance(node, ast.Name):
        if node.id in ctx:
            return ctx[node.id]
        raise NameError(node.id)
    if isinstance(node, ast.BinOp) and type(node.op) in _BINARY:
        return _BINARY[type(node.op)](_walk(node.left, ctx), _walk(node.right, ctx))
    if isinstance(node, ast.UnaryOp) and type(node.op) in _UNARY:
        return _UNARY[type(node.op)](_walk(node.operand, ctx))
    if isinstance(node, ast.Call) and not node.keywords:
        f = node.func
        name = f.id if isinstance(f, ast.Name) else (
            f.attr if isinstance(f, ast.Attribute) and isinstance(f.value, ast.Name) and f.value.id == "math"
            else None)
        if name in _CALLS:
            return _CALLS[name](*(_walk(a, ctx) for a in node.args))
    raise ValueError(f"unsupported expression element {ast.dump(node)[:60]}")


def _eval_expr(expr, ctx: dict) -> float | None:
    """A config's flops_expr / bytes_expr evaluated on a case (None when the
    expression is absent or cannot be evaluated on it)."""
    if expr is None or str(expr).strip() == "":
        return None
    try:
        return float(_walk(ast.parse(str(expr), mode="eval"), ctx))
    except (ArithmeticError, NameError, SyntaxError, TypeError, ValueError):
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
    """Backends whose throughput may be set against `peak_cfg`: the file's own
    "backends" list when it has one, else every backend that runs on a GPU."""
    listed = tuple((peak_cfg or {}).get("backends") or ())
    return listed or tuple(b for b in BACKENDS if b not in NON_GPU_BACKENDS)


def _bw_peak(cfg: dict, metrics_cfg: dict) -> float | None:
    v = (cfg or {}).get("peak_bw_GBs") or metrics_cfg.get("peak_bw_GBs")
    return None if v is None else float(v)


def _matrix_peak(cfg: dict, key: str | None) -> float | None:
    """The matrix peak named `key` ("fp16", "fp16_mma", "int8" ...): the
    calibration files name them with an "_mma" suffix, the published ones
    without it."""
    if not key:
        return None
    table = {**((cfg or {}).get("peak_tops") or {}), **((cfg or {}).get("peak_tflops") or {})}
    base = key[:-4] if key.endswith("_mma") else key
    for k in (key, f"{base}_mma", base):
        if k in table and table[k] is not None:
            return float(table[k])
    return None


def compute_derived(result: dict, metrics_cfg: dict, peak_cfg: dict | None = None,
                    calibrated_cfg: dict | None = None) -> dict:
    """Per-backend latency, GB/s, TFLOPS, % of peak, AI and speedup over torch.

    pct_peak_bw / pct_peak_tflops are against `peak_cfg` (published peaks);
    pct_calibrated_peak_bw / pct_calibrated_peak_tflops against
    `calibrated_cfg` when given."""
    flops, nbytes = work(metrics_cfg, result.get("params", {}), result.get("dtype", "fp32"))
    mode = metrics_cfg.get("peak_tflops_key") or result.get("dtype")
    refs = {"": peak_cfg or {}, "calibrated_": calibrated_cfg or {}}
    peaks = {tag: (_bw_peak(cfg, metrics_cfg if tag == "" else {}), _matrix_peak(cfg, mode))
             for tag, cfg in refs.items()}
    torch_ms = result.get("torch_ms")
    base_ms = float(torch_ms) if torch_ms is not None and float(torch_ms) > 0 else None
    out = {}
    for backend in BACKENDS:
        ms = result.get(f"{backend}_ms")
        if ms is None or not float(ms) > 0:
            continue
        sec = float(ms) * 1e-3
        d = {"latency_ms": float(ms)}
        if nbytes:
            d["bandwidth_GBs"] = nbytes / sec / 1e9
        if flops:
            d["tflops"] = flops / sec / 1e12
        if flops and nbytes:
            d["arithmetic_intensity"] = flops / nbytes
        for tag, (bw, tf) in peaks.items():
            if backend not in applicable_backends(refs[tag]):
                continue
            if bw and "bandwidth_GBs" in d:
                d[f"pct_{tag}peak_bw"] = 100.0 * d["bandwidth_GBs"] / bw
            if tf and "tflops" in d:
                d[f"pct_{tag}peak_tflops"] = 100.0 * d["tflops"] / tf
        if backend != "torch" and base_ms is not None:
            d["speedup"] = base_ms / float(ms)
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
