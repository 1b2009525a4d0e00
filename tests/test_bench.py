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
    monkeypatch.setattr(bench, "calibrated_peak", lambda bound, key: 1600.0)
    w = {"bound": "mfma", "flops": 2e12, "bytes": 1, "peak_key": "fp16", "kernel": "tb::w4a16::w4a16_prefill"}
    r = bench.roofline(w, 1.0)  # 2e12 flop in 1 ms = 2000 TFLOP/s
    assert r["unit"] == "TFLOP/s" and r["achieved"] == 2000.0
    assert r["peak"] == 2500.0 and r["frac"] == 0.8
    assert r["measured_peak"] == 2000.0 and r["frac_of_measured"] == 1.0
    assert r["calibrated_peak"] == 1600.0 and r["frac_of_calibrated"] == 1.25
    # the committed rocprofv3 FETCH_SIZE + WRITE_SIZE summary of this kernel
    assert isinstance(r["traffic"], int) and r["traffic"] > 0
    assert r["kernel"] == "tb::w4a16::w4a16_prefill"


def test_roofline_hbm_bound_and_unmeasured_peak(monkeypatch):
    seen = []
    monkeypatch.setattr(bench, "measured_peak", lambda bound, key: seen.append((bound, key)) or None)
    monkeypatch.setattr(bench, "calibrated_peak", lambda bound, key: None)
    w = {"bound": "hbm", "flops": None, "bytes": 4e9, "peak_key": None, "kernel": "no::such_kernel"}
    r = bench.roofline(w, 1.0)  # 4 GB in 1 ms = 4000 GB/s
    assert seen == [("hbm", None)]
    assert r["unit"] == "GB/s" and r["achieved"] == 4000.0 and r["frac"] == 0.5
    assert r["measured_peak"] is None and r["frac_of_measured"] is None
    assert r["traffic"] is None


def test_more_than_one_gpu_is_refused(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU" in capsys.readouterr().err


def test_input_sets_cover_twice_the_mall():
    """Small workloads get enough copies that a timed set is reused only after
    the steps on the other sets have moved 2x the 256 MiB MALL, and the warm
    sets are distinct."""
    import torch
    x = (torch.zeros(4 * 1024 * 1024 // 4, dtype=torch.float32), 64, 8)   # 4 MiB of input
    w = {"out_bytes": 1024 * 1024}                                          # + 1 MiB of output per step
    timed, warm = bench.input_sets(w, x, steps=20)
    per = 5 * 1024 * 1024
    assert len(timed) == 20            # fewer steps than the rotation: no timed set is used twice
    assert (len(warm) - 1) * per >= 2 * bench.MALL_BYTES
    ptrs = {s[0].data_ptr() for s in timed + warm}
    assert len(ptrs) == len(timed) + len(warm)
    assert all(s[1:] == (64, 8) for s in timed + warm)
    # the headline's traffic (147 MB per step): each set comes back after steps on the
    # others that move >= 2x the MALL
    per = 147_156_992
    x = (torch.zeros(per // 2, dtype=torch.uint8),)
    timed, warm = bench.input_sets({"out_bytes": per - per // 2}, x, steps=20)
    assert (len(timed) - 1) * per >= 2 * bench.MALL_BYTES and (len(warm) - 1) * per >= 2 * bench.MALL_BYTES
    # a step that already moves more than 2x the MALL: two sets alternate
    big = (torch.zeros(1, dtype=torch.uint8),)
    timed, warm = bench.input_sets({"out_bytes": 4 * bench.MALL_BYTES}, big, steps=100)
    assert len(timed) == 2 and len(warm) == 2


def test_fp32_matmul_is_priced_as_bf16_mfma_work(monkeypatch):
    monkeypatch.setattr(bench, "measured_peak", lambda bound, key: None)
    monkeypatch.setattr(bench, "calibrated_peak", lambda bound, key: None)
    w = {"bound": "mfma", "flops": 1e12, "mfma_flops": 3e12, "bytes": 1, "peak_key": "bf16",
         "kernel": "tb::ntg::nt_gemm<2, 3, 256, 256, 128, 64>"}
    r = bench.roofline(w, 2.0)          # 3e12 bf16 flop in 2 ms = 1500 TFLOP/s
    assert r["achieved"] == 1500.0 and r["peak"] == 2500.0 and r["frac"] == 0.6
    assert "500.00 TFLOP/s" in r["note"]


def test_cpu_baseline_is_the_torch_reference_with_every_core():
    import torch
    calls = []
    w = {"unit": "GB/s", "cpu": lambda: ((lambda: calls.append(torch.get_num_threads())), 2e9, "tiny")}
    before = torch.get_num_threads()
    r = bench.cpu_baseline(w)
    assert len(calls) == 4                               # warmup 1 + repeat 3
    assert set(calls) == {r["cores"]} and r["cores"] == bench._host_cores()
    assert torch.get_num_threads() == before             # restored afterwards
    assert r["kind"] == "port" and r["impl"] == "torch" and r["unit"] == "GB/s"
    assert "warmup 1, repeat 3" in r["sample"] and r["cpu_model"]
