"""Checks the eviction size the timer flushes against the device's last-level cache.

The timer evicts the cache before every timed launch by storing over a buffer of
2x the last-level cache (tilebench_amd/hardware.py registers 256 MiB of MALL for
cdna4, the datasheet figure; the reference's rule is tilebench/core/timer.py:81-104).
This sweep measures where that cache ends: tb_probe_copy moves a working set of
S bytes (S/2 read, S/2 written) back to back, so a working set that fits in the
cache is served from it on every launch after the first ("warm"), and each size
is also timed as single launches, each after a synchronisation, once without
and once right after tb_l2_flush, the timer's own flush.  Single launches with
and without the flush differ only in what the cache holds, so their gap is the
cache's benefit and shows whether the flush evicts.  The back-to-back rate falls
where S passes the cache size, if the cache serves a streaming copy faster than
HBM does.

Usage:  python -m tilebench_amd.profiling.mall_sweep --out profiles/mall_sweep_MI355X.txt
"""
from __future__ import annotations

import argparse
import statistics
import sys

import torch

from tilebench_amd import hardware
from tilebench_amd import runtime as rt
from tilebench_amd.core.timer import _flush_l2_buffer_mb, flush_l2_cache

MIB = 1024 * 1024
SIZES_MIB = (16, 32, 64, 96, 128, 160, 192, 224, 256, 288, 320, 384, 512, 768, 1024)


def _time_copy(src: torch.Tensor, dst: torch.Tensor, launches: int, flush: bool, samples_n: int = 1) -> float:
    """Median over samples of the mean microseconds per tb_probe_copy launch."""
    stream = rt.stream_handle()
    nbytes = src.numel()
    samples = []
    for _ in range(samples_n):
        if flush:
            flush_l2_cache()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(launches):
            rt.call("tb_probe_copy", src.data_ptr(), dst.data_ptr(), nbytes, stream)
        e1.record()
        torch.cuda.synchronize()
        samples.append(e0.elapsed_time(e1) * 1000.0 / launches)
    return statistics.median(samples)


def sweep(sizes_mib=SIZES_MIB) -> list[dict]:
    rt.require_device()
    rows = []
    for s in sizes_mib:
        buf = torch.empty(s * MIB, dtype=torch.uint8, device="cuda")
        half = s * MIB // 2
        src, dst = buf[:half], buf[half:]
        for _ in range(3):
            rt.call("tb_probe_copy", src.data_ptr(), dst.data_ptr(), half, rt.stream_handle())
        warm = _time_copy(src, dst, 20, flush=False)
        single = _time_copy(src, dst, 1, flush=False, samples_n=5)
        cold = _time_copy(src, dst, 1, flush=True, samples_n=5)
        rows.append({"working_set_mib": s, "warm_us": warm, "warm_tbs": s * MIB / warm / 1e6,
                     "single_us": single, "single_tbs": s * MIB / single / 1e6,
                     "cold_us": cold, "cold_tbs": s * MIB / cold / 1e6})
        print(f"{s:5d} MiB  back-to-back {warm:8.1f} us {rows[-1]['warm_tbs']:5.2f} TB/s   "
              f"single {single:8.1f} us {rows[-1]['single_tbs']:5.2f} TB/s   "
              f"after flush {cold:8.1f} us {rows[-1]['cold_tbs']:5.2f} TB/s", flush=True)
        del buf, src, dst
        torch.cuda.empty_cache()
    return rows


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--out", default=None, help="write the table (text) here")
    args = ap.parse_args(argv)
    arch = hardware.detect_arch()
    llc = hardware.last_level_cache_bytes()
    print(f"arch {arch}; registered last-level cache {llc // MIB if llc else None} MiB; "
          f"flush buffer {_flush_l2_buffer_mb()} MiB", flush=True)
    rows = sweep()
    if args.out:
        with open(args.out, "w") as f:
            f.write("# MALL size check: tb_probe_copy rate against working set (MI355X, one GPU)\n\n")
            f.write("Command:\n  python -m tilebench_amd.profiling.mall_sweep --out " + args.out + "\n\n")
            f.write(f"arch {arch}; registered last-level cache {llc // MIB if llc else None} MiB; flush buffer "
                    f"{_flush_l2_buffer_mb()} MiB.  Working set S = S/2 read + S/2 written per launch.\n"
                    "back-to-back: mean of 20 launches after 3 untimed ones; single: median of 5 single\n"
                    "launches, each after a synchronisation; flushed: the same, each right after tb_l2_flush\n"
                    "over the flush buffer.\n\n")
            f.write("working_set_MiB  b2b_us  b2b_TB/s  single_us  single_TB/s  flushed_us  flushed_TB/s\n")
            for r in rows:
                f.write(f"{r['working_set_mib']:15d} {r['warm_us']:7.1f} {r['warm_tbs']:9.2f} {r['single_us']:10.1f} "
                        f"{r['single_tbs']:12.2f} {r['cold_us']:11.1f} {r['cold_tbs']:13.2f}\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
