"""Kernel timing: hipGraph replay, hipEvent timing and an explicit cache flush.

Replaces the reference's Proton-based timer (tilebench/core/timer.py:208
``report_benchmark``), which on ROCm cannot attribute graph child kernels and
falls back to eager launches (timer.py:53-63).  Here, per timed sample:

    [flush: fill a 2 x LLC buffer with a store kernel]
    [hipEventRecord(start); hipGraphLaunch(run); hipEventRecord(stop)]

all on the current stream, with the flush outside the events.  ``run`` is
captured once into a hipGraph (torch.cuda.CUDAGraph is hipGraph on ROCm) after
the warmup launches; a callable that cannot be captured is timed eagerly and
the result says so.  Samples are kept individually, as in the reference's
evaluation timer (tilebench/llm/v2/evaluation/timing.py:87-161).
"""
from __future__ import annotations

import statistics
from typing import Any, Callable

import torch

from tilebench_amd.hardware import last_level_cache_bytes

#: Formal protocol when neither config.yaml nor the CLI sets one (timer.py:43-44).
DEFAULT_WARMUP = 1
DEFAULT_REPEAT = 3

_flush_buf: torch.Tensor | None = None


def _flush_l2_buffer_mb() -> int:
    """Eviction buffer: 2x the device's last-level cache (the reference's rule,
    timer.py:81-104); on MI355X 2 x 256 MiB MALL = 512 MiB."""
    llc = last_level_cache_bytes()
    if llc is None:
        llc = 128 * 1024 * 1024
    return max(64, 2 * llc // (1024 * 1024))


def flush_l2_cache(flush_mb: int | None = None) -> None:
    """Enqueue a store sweep over the eviction buffer on the current stream
    (asynchronous; the next kernel on the stream starts with a cold cache)."""
    from tilebench_amd import runtime as rt

    global _flush_buf
    nbytes = (flush_mb or _flush_l2_buffer_mb()) * 1024 * 1024
    if _flush_buf is None or _flush_buf.numel() * 4 != nbytes:
        _flush_buf = torch.empty(nbytes // 4, device="cuda", dtype=torch.float32)
    rt.call("tb_l2_flush", _flush_buf.data_ptr(), nbytes, 0x3F800000, rt.stream_handle())


def effective_use_cuda_graph(requested: bool) -> bool:
    """Graph replay is honoured on ROCm too: events bracket the replay, so no
    tracer has to attribute the graph's child kernels."""
    return bool(requested)


def timing_mode(requested: bool) -> dict[str, Any]:
    eff = effective_use_cuda_graph(requested)
    return {"requested_use_cuda_graph": bool(requested), "effective_use_cuda_graph": eff,
            "timing_execution_mode": "graph" if eff else "eager", "timing_note": None}


def _capture(f: Callable, args: tuple, kwargs: dict):
    """Capture one call of f into a graph; returns a replay callable or None."""
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_out = f(*args, **kwargs)

        def replay():
            graph.replay()
            return static_out

        replay.graph = graph  # keep the graph (and its pool) alive with the runner
        return replay
    except Exception:
        torch.cuda.synchronize()
        return None


def report_benchmark(f: Callable[..., Any], tuple_of_args: tuple, kwargs: dict | None = None, *,
                     warmup: int = DEFAULT_WARMUP, repeat: int = DEFAULT_REPEAT, use_cuda_graph: bool = True,
                     flush_l2: bool = True, **_unused) -> dict:
    """Mean device time (ms) of f(*args) over `repeat` samples.

    Returns {"mean", "median", "min", "max", "samples", "mode", "flush_mb"}."""
    kwargs = kwargs or {}
    flush_mb = _flush_l2_buffer_mb() if flush_l2 else 0
    for _ in range(max(0, warmup)):
        if flush_l2:
            flush_l2_cache(flush_mb)
        f(*tuple_of_args, **kwargs)
    torch.cuda.synchronize()

    runner = _capture(f, tuple_of_args, kwargs) if effective_use_cuda_graph(use_cuda_graph) else None
    mode = "graph" if runner is not None else "eager"
    if runner is None:
        def runner():
            return f(*tuple_of_args, **kwargs)
    else:
        runner()  # first replay uploads the graph
    torch.cuda.synchronize()

    n = max(1, repeat)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    stops = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for i in range(n):
        if flush_l2:
            flush_l2_cache(flush_mb)
        starts[i].record()
        runner()
        stops[i].record()
    torch.cuda.synchronize()
    samples = [s.elapsed_time(e) for s, e in zip(starts, stops)]
    return {"mean": sum(samples) / n, "median": statistics.median(samples), "min": min(samples),
            "max": max(samples), "samples": samples, "mode": mode, "flush_mb": flush_mb}
