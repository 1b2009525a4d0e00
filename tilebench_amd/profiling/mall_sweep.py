"""Eviction sweep: how large a flush the timer needs to start a launch cold.

The timer stores over a buffer of 2x the last-level cache before every timed
launch (the reference's rule, tilebench/core/timer.py:81-104), and
tilebench_amd/hardware.py registers that cache's size per architecture.  The
reference validates its entry the way this sweep does
(tilebench/hardware.py:24-37): a fixed re-read probe behind flushes of growing
size.  The probe reads a P-byte buffer with plain loads (tb_probe_read).  For
each flush size F, a sample is: read the buffer once (it is now as warm as the
caches can make it), flush F bytes, then time one more read with hipEvents.
While F is below what the caches hold, part of the buffer survives and the
timed read is faster; from the eviction size on, the read is as slow as the
cold reference (the first read of the buffer after a 2 GiB flush).  Two
flushes are swept: tb_l2_flush (the timer's store kernel, nontemporal stores)
and torch's fill_ (plain stores).

Usage:  python -m tilebench_amd.profiling.mall_sweep --out profiles/mall_sweep_MI355X.txt
"""
from __future__ import annotations

import argparse
import statistics
import sys

import torch

from tilebench_amd import hardware
from tilebench_amd import runtime as rt
from tilebench_amd.core.timer import _flush_l2_buffer_mb

MIB = 1024 * 1024
PROBE_MIB = (64, 128)
FLUSH_MIB = (0, 16, 32, 64, 96, 128, 160, 192, 224, 256, 320, 384, 512, 768, 1024)
KEY = 0xDEADBEEF  # the probe buffer is all zeros: no granule XORs to this


def _read_us(probe: torch.Tensor, sink: torch.Tensor, flush, reps: int = 7) -> float:
    """Median microseconds of one probe read placed right after `flush()`."""
    stream = rt.stream_handle()
    times = []
    for _ in range(reps):
        rt.call("tb_probe_read", probe.data_ptr(), probe.numel(), KEY, sink.data_ptr(), stream)  # warm it
        flush()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        rt.call("tb_probe_read", probe.data_ptr(), probe.numel(), KEY, sink.data_ptr(), stream)
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1000.0)
    return statistics.median(times)


def sweep(probe_mib=PROBE_MIB, flush_mib=FLUSH_MIB) -> dict:
    rt.require_device()
    stream = rt.stream_handle()
    big = torch.empty(max(max(flush_mib), 2048) * MIB, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4, dtype=torch.uint32, device="cuda")

    def nt_flush(nbytes):
        return (lambda: None) if nbytes == 0 else \
            (lambda: rt.call("tb_l2_flush", big.data_ptr(), nbytes, 0x3F800000, stream))

    def fill_flush(nbytes):
        view = big[:nbytes]
        return (lambda: None) if nbytes == 0 else (lambda: view.fill_(0x5A))

    out = {"probes": []}
    for p in probe_mib:
        probe = torch.zeros(p * MIB, dtype=torch.uint8, device="cuda")
        cold_flush = nt_flush(2048 * MIB)
        cold = _read_us(probe, sink, cold_flush)
        rows = []
        for f in flush_mib:
            nt = _read_us(probe, sink, nt_flush(f * MIB))
            pl = _read_us(probe, sink, fill_flush(f * MIB))
            rows.append({"flush_mib": f, "nt_us": nt, "fill_us": pl})
            print(f"probe {p:4d} MiB  flush {f:5d} MiB   after tb_l2_flush {nt:7.2f} us ({p * MIB / nt / 1e6:5.2f} TB/s)"
                  f"   after fill_ {pl:7.2f} us ({p * MIB / pl / 1e6:5.2f} TB/s)   cold {cold:7.2f} us", flush=True)
        out["probes"].append({"probe_mib": p, "cold_us": cold, "rows": rows})
        del probe
        torch.cuda.empty_cache()
    del big
    torch.cuda.empty_cache()
    return out


def eviction_size(probe: dict, tol: float = 0.03) -> dict:
    """Smallest flush (per flush kind) from which every larger flush leaves the
    probe read within `tol` of the cold read; None if no flush gets there."""
    res = {}
    for kind in ("nt_us", "fill_us"):
        cold = probe["cold_us"]
        ok = [r[kind] >= cold * (1 - tol) for r in probe["rows"]]
        first = None
        for i in range(len(ok)):
            if all(ok[i:]):
                first = probe["rows"][i]["flush_mib"]
                break
        res[kind[:-3]] = first
    return res


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--out", default=None, help="write the table (text) here")
    args = ap.parse_args(argv)
    arch = hardware.detect_arch()
    llc = hardware.last_level_cache_bytes()
    head = (f"arch {arch}; registered last-level cache {llc // MIB if llc else None} MiB; "
            f"timer flush buffer {_flush_l2_buffer_mb()} MiB")
    print(head, flush=True)
    res = sweep()
    lines = [head, "",
             "Each cell: median of 7 samples of [read the probe buffer; flush F MiB; time one read of it].",
             "cold: the same read after a 2048 MiB flush.  Probe data all zeros (plain loads, tb_probe_read).", ""]
    for p in res["probes"]:
        ev = eviction_size(p)
        lines.append(f"probe {p['probe_mib']} MiB, cold read {p['cold_us']:.2f} us "
                     f"({p['probe_mib'] * MIB / p['cold_us'] / 1e6:.2f} TB/s); cold (within 3 %) from a flush of "
                     f"{ev['nt']} MiB (tb_l2_flush) / {ev['fill']} MiB (fill_)")
        lines.append("flush_MiB  after_tb_l2_flush_us  after_fill_us")
        for r in p["rows"]:
            lines.append(f"{r['flush_mib']:9d}  {r['nt_us']:20.2f}  {r['fill_us']:13.2f}")
        lines.append("")
    text = "\n".join(lines) + "\n"
    print(text, flush=True)
    if args.out:
        with open(args.out, "w") as f:
            f.write("# Eviction sweep (MI355X): a fixed re-read probe behind flushes of growing size\n\n")
            f.write("Command:\n  python -m tilebench_amd.profiling.mall_sweep --out " + args.out + "\n\n")
            f.write(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
