"""Kernel timing: hipGraph replay, hipEvent timing and an explicit cache flush.

Replaces the reference's Proton-based timer (tilebench/core/timer.py:208
``report_benchmark``), which on ROCm cannot attribute graph child kernels and
falls back to eager launches (timer.py:53-63).  Here, per timed sample:

    [flush: store over a 2 x LLC buffer with tb_l2_flush]
    [hipEventRecord(start); hipGraphLaunch(run); hipEventRecord(stop)]

all on the current stream, with the flush outside the events.  ``run`` is
captured once into a hipGraph (torch.cuda.CUDAGraph is hipGraph on ROCm) after
the warmup launches; a callable that cannot be captured is timed eagerly and
the result says so.  Samples are kept individually, as in the reference's
evaluation timer (tilebench/llm/v2/evaluation/timing.py:87-161).

Two times come out of every sample:
  * the device time of run()'s kernels, read from the kernels' own start and
    end timestamps (torch.profiler's ROCm activity records, the source rocprof
    reads too).  This is what Proton reports in the reference, so it is the
    result's ``mean``;
  * the hipEvent bracket of the graph replay (``event_*``).  On MI355X a replay
    costs about 10 us more than its kernels: the graph's closing release makes
    the L2's dirty lines visible to the host.  For a microsecond kernel that
    fixed cost is larger than the kernel, so it is reported, not used as the
    result.
A profiled run whose records miss a kernel (the tracer reads its buffers
asynchronously) is run again, up to TIMESTAMP_ATTEMPTS times in all.
Without the activity records (profiler unavailable), or with an external
rocprofiler tool attached to the process (rocprofv3 sets ROCP_TOOL_LIBRARIES;
torch's activity records are then not trustworthy), ``mean`` falls back to the
event bracket and ``time_source`` says so.
"""
from __future__ import annotations

import os
import statistics
from typing import Any, Callable

import torch

from tilebench_amd.hardware import last_level_cache_bytes

#: Formal protocol when neither config.yaml nor the CLI sets one (timer.py:43-44).
DEFAULT_WARMUP = 1
DEFAULT_REPEAT = 3

#: name fragment of the flush kernel (tb_l2_flush), told apart from run()'s kernels
FLUSH_KERNEL = "fill_kernel"
#: profiled runs tried before the events alone time a call
TIMESTAMP_ATTEMPTS = 3

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
    """Graph replay is honoured on ROCm too: events bracket the replay and the
    kernels' own timestamps are read per sample, so no tracer has to attribute
    the graph's child kernels to a scope."""
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


def kernel_times_per_sample(kernels: list[tuple[str, float, float]], n: int, flushed: bool) -> list[float] | None:
    """Split device kernel records (name, start_us, duration_us), in start
    order, into the n samples and return each sample's kernel time in ms.

    With a flush, every sample starts at a flush kernel and holds the kernels
    up to the next one; without, the records must split evenly into n runs.
    None when the records do not match the samples (nothing recorded, or a
    count that does not divide)."""
    if not kernels:
        return None
    if flushed:
        groups: list[list[float]] = []
        for name, _start, dur in kernels:
            if FLUSH_KERNEL in name:
                groups.append([])
            elif groups:
                groups[-1].append(dur)
        if len(groups) != n or any(not g for g in groups):
            return None
        return [sum(g) / 1e3 for g in groups]
    if len(kernels) % n:
        return None
    per = len(kernels) // n
    return [sum(d for _, _, d in kernels[i * per:(i + 1) * per]) / 1e3 for i in range(n)]


def _device_kernels(prof) -> list[tuple[str, float, float]]:
    out = []
    for e in prof.events():
        if e.device_type != torch.autograd.DeviceType.CUDA:
            continue
        tr = getattr(e, "time_range", None)
        if tr is None:
            continue
        out.append((e.name, float(tr.start), float(tr.end - tr.start)))
    out.sort(key=lambda k: k[1])
    return out


def external_profiler_attached() -> bool:
    """True when a rocprofiler-sdk tool (rocprofv3) runs inside this process."""
    return bool(os.environ.get("ROCP_TOOL_LIBRARIES"))


def report_benchmark(f: Callable[..., Any], tuple_of_args: tuple, kwargs: dict | None = None, *,
                     warmup: int = DEFAULT_WARMUP, repeat: int = DEFAULT_REPEAT, use_cuda_graph: bool = True,
                     flush_l2: bool = True, kernel_timestamps: bool = True, **_unused) -> dict:
    """Mean device time (ms) of f(*args) over `repeat` samples.

    Returns {"mean", "median", "min", "max", "samples", "time_source",
    "event_mean", "event_samples", "mode", "flush_mb"}: `samples` are the
    kernels' device time per sample when their timestamps were read, else the
    event brackets."""
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

    def sample_all():
        for i in range(n):
            if flush_l2:
                flush_l2_cache(flush_mb)
            starts[i].record()
            runner()
            stops[i].record()
        torch.cuda.synchronize()

    kernel_ms = None
    attempts = 0
    if kernel_timestamps and not external_profiler_attached():
        # The activity records of a profiled run now and then miss a kernel
        # (the tracer's buffers are read asynchronously); such a run is timed
        # again, up to TIMESTAMP_ATTEMPTS times, before the events alone are used.
        try:
            from torch.profiler import ProfilerActivity, profile

            while kernel_ms is None and attempts < TIMESTAMP_ATTEMPTS:
                attempts += 1
                with profile(activities=[ProfilerActivity.CUDA]) as prof:
                    sample_all()
                kernel_ms = kernel_times_per_sample(_device_kernels(prof), n, flush_l2)
        except Exception:  # no activity records here: time with the events alone
            torch.cuda.synchronize()
            kernel_ms = None
            sample_all()
    else:
        sample_all()
    events = [s.elapsed_time(e) for s, e in zip(starts, stops)]
    samples = kernel_ms if kernel_ms is not None else events
    return {"mean": sum(samples) / n, "median": statistics.median(samples), "min": min(samples),
            "max": max(samples), "samples": samples,
            "time_source": ("kernel timestamps" if kernel_ms is not None else
                            "hipEvents (rocprofiler tool attached)" if external_profiler_attached() else "hipEvents"),
            "timestamp_attempts": attempts,
            "event_mean": sum(events) / n, "event_samples": events, "mode": mode, "flush_mb": flush_mb}
