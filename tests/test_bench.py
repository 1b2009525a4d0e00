"""bench.py's report fields on the host: roofline fractions against the
published and the measured peak, the committed traffic lookup, and the
one-GPU guard.  No GPU: the measured peak is stubbed."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_roofline_fractions_of_published_and_measured_peak(monkeypatch):
    monkeypatch.setattr(bench, "measured_peak", lambda bound, key: 2000.0)
    w = {"bound": "mfma", "flops": 2e12, "bytes": 1, "peak_key": "fp16", "kernel": "tb::w4a16::w4a16_prefill"}
    r = bench.roofline(w, 1.0)  # 2e12 flop in 1 ms = 2000 TFLOP/s
    assert r["unit"] == "TFLOP/s" and r["achieved"] == 2000.0
    assert r["peak"] == 2500.0 and r["frac"] == 0.8
    assert r["measured_peak"] == 2000.0 and r["frac_of_measured"] == 1.0
    # the committed rocprofv3 FETCH_SIZE + WRITE_SIZE summary of this kernel
    assert isinstance(r["traffic"], int) and r["traffic"] > 0
    assert r["kernel"] == "tb::w4a16::w4a16_prefill"


def test_roofline_hbm_bound_and_unmeasured_peak(monkeypatch):
    seen = []
    monkeypatch.setattr(bench, "measured_peak", lambda bound, key: seen.append((bound, key)) or None)
    w = {"bound": "hbm", "flops": None, "bytes": 4e9, "peak_key": None, "kernel": "no::such_kernel"}
    r = bench.roofline(w, 1.0)  # 4 GB in 1 ms = 4000 GB/s
    assert seen == [("hbm", None)]
    assert r["unit"] == "GB/s" and r["achieved"] == 4000.0 and r["frac"] == 0.5
    assert r["measured_peak"] is None and r["frac_of_measured"] is None
    assert r["traffic"] is None


def test_more_than_one_gpu_is_refused(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU" in capsys.readouterr().err
