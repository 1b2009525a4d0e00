"""Per-case benchmark harness.

Same flow and result schema as tilebench/core/engine.py:103-500
(``run_benchmark_suite``): load the operator's config.yaml, import
``impl_torch`` and one ``impl_<backend>`` module per selected backend (an
ImportError skips that backend), expand the case grid, and for each case
generate inputs, run the torch reference, then run, verify and — only when
verified — time each backend.  The reference hard-codes one block per backend
(engine.py:337-459); here one loop covers every name in BACKEND_ORDER, so the
``hip`` backend is driven by exactly the code that drives the others.
"""
from __future__ import annotations

import importlib
import inspect
import math

import torch
import yaml

from tilebench_amd.backends import BACKEND_ORDER
from tilebench_amd.core.dtypes import resolve_dtype
from tilebench_amd.core.timer import DEFAULT_REPEAT, DEFAULT_WARMUP, report_benchmark, timing_mode
from tilebench_amd.core.verifier import config_per_output, config_tolerance, verify
from tilebench_amd.data.tensors import expand_cases, get_generator, infer_problem_size
from tilebench_amd.hardware import detect_arch
from tilebench_amd.paths import operator_config

HAS_CUDA = torch.cuda.is_available()
DEFAULT_ENABLED_BACKENDS = BACKEND_ORDER


def _sync():
    if HAS_CUDA:
        torch.cuda.synchronize()


def _to_device(x, device):
    """Tensors of a (nested) tuple moved to `device`; other values as they are."""
    if isinstance(x, torch.Tensor):
        return x.to(device)
    if isinstance(x, (tuple, list)):
        return type(x)(_to_device(v, device) for v in x)
    return x


def _device_of(inputs):
    for v in inputs:
        if isinstance(v, torch.Tensor):
            return v.device
    return torch.device("cpu")


def _import_impl(operator_name: str, backend: str):
    """The backend's module, or None (with the reason printed) when it cannot load."""
    try:
        return importlib.import_module(f"tilebench_amd.benchmarks.operators.{operator_name}.impl_{backend}")
    except ImportError as e:
        print(f"  {backend} import skipped: {e}")
        return None


def _run_kwargs(fn, block_size, autotune):
    sig = inspect.signature(fn).parameters
    kw = {}
    if "block_size" in sig:
        kw["block_size"] = block_size
    if "autotune" in sig:
        kw["autotune"] = autotune
    return kw


def run_benchmark_suite(operator_name, benchmark_overrides=None, enabled_backends=None, logs_dir=None,
                        bench_fn=None):
    """Run every case of `operator_name`; returns one result dict per case.

    bench_fn (default core.timer.report_benchmark) may be replaced, as the
    reference's tests monkeypatch engine.report_benchmark."""
    bench_fn = bench_fn or report_benchmark
    with open(operator_config(operator_name)) as f:
        config = yaml.safe_load(f)
    enabled = set(DEFAULT_ENABLED_BACKENDS if enabled_backends is None else enabled_backends)

    impl_torch = importlib.import_module(f"tilebench_amd.benchmarks.operators.{operator_name}.impl_torch")
    impls = {}
    for b in BACKEND_ORDER:
        if b in enabled:
            impls[b] = _import_impl(operator_name, b)
        else:
            impls[b] = None
            print(f"  {b} not selected (--tile-language)")
    generate_inputs = get_generator(operator_name)

    bench_cfg = dict(config.get("benchmark", {}))
    bench_cfg.update(benchmark_overrides or {})
    grid = bench_cfg.get("grid")
    if grid is not None:
        # a named alternative grid of the same operator (config "grids:" entry),
        # e.g. the reference's own case grid beside the BASELINE one
        alt = (config.get("grids") or {}).get(grid)
        if alt is None:
            raise ValueError(f"{operator_name}: no grid named {grid!r} in config.yaml (have "
                             f"{sorted(config.get('grids') or {})})")
        config = {k: v for k, v in config.items() if k not in ("case_grid", "case_defaults", "test_cases")}
        config.update(alt)  # its own case_defaults / case_grid (and verify, if it sets one)
    warmup = int(bench_cfg.get("warmup", DEFAULT_WARMUP))
    repeat = int(bench_cfg.get("repeat", DEFAULT_REPEAT))
    autotune = bool(bench_cfg.get("autotune", False))
    use_graph = bool(bench_cfg.get("use_cuda_graph", True))
    flush_l2 = bool(bench_cfg.get("flush_l2", True))
    verify_cfg = config.get("verify", {}) or {}
    arch = detect_arch()
    atol, rtol = config_tolerance(verify_cfg, arch)
    per_output = config_per_output(verify_cfg, arch)
    # verify.reference_device: cpu runs the torch reference on CPU copies of the
    # inputs (its IEEE arithmetic) for the correctness check; torch_ms still
    # times it on the GPU inputs
    ref_on_cpu = str(verify_cfg.get("reference_device", "")).lower() == "cpu"
    timing = timing_mode(use_graph) if HAS_CUDA else None

    cases = expand_cases(operator_name, config)
    if bench_cfg.get("case_indices") is not None:
        idxs = list(bench_cfg["case_indices"])
        for i in idxs:
            if i < 0 or i >= len(cases):
                raise ValueError(f"case index {i} out of range for {len(cases)} generated cases")
        cases = [cases[i] for i in idxs]
    if bench_cfg.get("case_overrides"):
        cases = [{**c, **bench_cfg["case_overrides"]} for c in cases]

    def _bench(impl, fn, args, kw):
        prepare = getattr(impl, "prepare_timed_run", None) if impl is not None else None
        if prepare is not None:
            launch, restore = prepare(*args, **kw)

            def _prepared():
                restore()
                return launch()
            return bench_fn(_prepared, (), {}, warmup=warmup, repeat=repeat, use_cuda_graph=use_graph,
                            flush_l2=flush_l2)
        return bench_fn(fn, args, kw, warmup=warmup, repeat=repeat, use_cuda_graph=use_graph, flush_l2=flush_l2)

    results = []
    for case in cases:
        params = {k: v for k, v in case.items() if k not in ("dtype", "block_size")}
        dtype_str = case.get("dtype", "fp32")
        dtype = resolve_dtype(dtype_str)
        block_size = case.get("block_size", 1024)
        print(f"Running case: {params}, dtype={dtype_str}")
        try:
            inputs = generate_inputs(**params, dtype=dtype)
        except (RuntimeError, TypeError, ValueError) as e:
            print(f"  Skipped: input generation failed ({type(e).__name__}: {e})")
            continue
        try:
            if ref_on_cpu:
                ref_output = _to_device(impl_torch.run(*_to_device(inputs, "cpu")), _device_of(inputs))
            else:
                ref_output = impl_torch.run(*inputs)
            _sync()
        except (RuntimeError, TypeError, ValueError) as e:
            print(f"  Skipped: reference failed ({type(e).__name__}: {e})")
            continue

        row = {"params": params, "problem_size": infer_problem_size(operator_name, params), "dtype": dtype_str}
        if HAS_CUDA:
            torch_stats = _bench(None, impl_torch.run, inputs, {})
            row["torch_ms"], row["torch_stats"] = torch_stats["mean"], torch_stats
        else:
            row["torch_ms"], row["torch_stats"] = float("nan"), None

        for b in BACKEND_ORDER:
            impl = impls[b]
            ok, err, ms, stats, cfg = False, "", float("nan"), None, None
            if impl is None:
                err = f"{b} not available" if b in enabled else f"{b} not selected (--tile-language)"
            elif not HAS_CUDA:
                err = f"{b} requires a GPU"
            else:
                try:
                    kw = _run_kwargs(impl.run, block_size, autotune)
                    out = impl.run(*inputs, **kw)
                    _sync()
                    ok, err = verify(out, ref_output, atol=atol, rtol=rtol, per_output=per_output)
                    cfg = getattr(impl, "get_last_config", lambda: None)()
                    if not ok:
                        print(f"  {b} verification FAILED: {err}")
                    else:
                        stats = _bench(impl, impl.run, inputs, kw)
                        ms = stats["mean"]
                except Exception as e:  # a failing backend is recorded, never timed
                    ok, err, ms, stats = False, f"{type(e).__name__}: {e}", float("nan"), None
                    print(f"  {b} execution FAILED: {err}")
            row[f"{b}_ms"] = ms
            row[f"{b}_stats"] = stats or {}
            row[f"{b}_ok"] = ok
            row[f"{b}_err"] = err
            row[f"{b}_autotune_cfg"] = cfg if autotune else None
            row[f"{b}_config"] = cfg
            tm = row["torch_ms"]
            row[f"speedup_{b}"] = tm / ms if ms > 0 and not math.isnan(tm) else 0.0
        row["timing"] = timing
        results.append(row)
    return results
