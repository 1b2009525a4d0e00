"""Host-side harness tests (no GPU), in the reference's mock-first style
(tests/test_verify_tolerance.py, test_engine_case_skip.py, test_timing_policy.py,
test_hardware.py of Tilebench): fake backend modules injected into sys.modules,
a fake device, a fake timer."""
import sys
import types

import numpy as np
import pytest
import torch

from tilebench_amd import backends, hardware
from tilebench_amd.core import engine, metrics, timer, verifier
from tilebench_amd.data import tensors as T
from tilebench_amd.paths import list_operators, operator_config

# ----------------------------------------------------------------------------- backends


def test_backend_order_and_parsing():
    assert backends.BACKEND_ORDER[-1] == "hip" and "hip" in backends.GPU_BACKENDS
    assert backends.parse_backends(None) == list(backends.GPU_BACKENDS)
    assert backends.parse_backends("all") == list(backends.GPU_BACKENDS)
    assert backends.parse_backends("hip,torch") == ["hip"]
    assert backends.parse_backends("hip,triton") == ["triton", "hip"]
    assert backends.backend_tag(["hip", "triton"]) == backends.backend_tag(["triton", "hip"]) == "triton-hip"
    assert backends.backend_tag([]) == "torch"
    with pytest.raises(ValueError):
        backends.parse_backends("cuda")


# ----------------------------------------------------------------------------- verifier


def test_verify_bit_exact_mode_distinguishes_signed_zero_and_nan_codes():
    a = torch.tensor([0.0, 1.0], dtype=torch.float16)
    b = torch.tensor([-0.0, 1.0], dtype=torch.float16)
    ok, _ = verifier.verify(a, b, atol=1e-3, rtol=1e-3)
    assert ok
    ok, err = verifier.verify(a, b, atol=0, rtol=0)
    assert not ok and "bit-exact" in err
    q1 = torch.tensor([0x7F, 0x10], dtype=torch.uint8).view(torch.float8_e4m3fn)
    q2 = torch.tensor([0xFF, 0x10], dtype=torch.uint8).view(torch.float8_e4m3fn)
    assert not verifier.verify(q1, q2, atol=0, rtol=0)[0]
    assert verifier.verify(q1, q1.clone(), atol=0, rtol=0)[0]


def test_verify_per_output_tolerances():
    w = torch.tensor([[0.5, 0.5]])
    i = torch.tensor([[1, 2]], dtype=torch.int32)
    ref = (w + 5e-6, i)
    assert verifier.verify((w, i), ref, atol=1e-5, rtol=1e-5, per_output=[None, {"atol": 0, "rtol": 0}])[0]
    ok, err = verifier.verify((w, i + 1), ref, atol=1e-5, rtol=1e-5, per_output=[None, {"atol": 0, "rtol": 0}])
    assert not ok and err.startswith("output[1]")
    assert not verifier.verify((w,), ref)[0]                       # arity mismatch
    assert not verifier.verify(w.half(), w)[0]                     # dtype mismatch


def test_config_tolerance_arch_override():
    cfg = {"atol": 1e-2, "rtol": 1e-2, "arch_overrides": {"cdna4": {"atol": 5e-2}}}
    assert verifier.config_tolerance(cfg, "cdna3") == (1e-2, 1e-2)
    assert verifier.config_tolerance(cfg, "cdna4") == (5e-2, 1e-2)
    assert verifier.config_tolerance({}, None) == (None, None)


# ----------------------------------------------------------------------------- hardware


@pytest.fixture
def fake_device(monkeypatch):
    def install(arch, name="AMD Instinct MI355X"):
        hardware.device_info.cache_clear()
        hardware.detect_arch.cache_clear()
        props = types.SimpleNamespace(name=name, gcnArchName=arch, L2_cache_size=4 * 1024 * 1024)
        monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
        monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
        monkeypatch.setattr(torch.cuda, "get_device_properties", lambda i: props)
        monkeypatch.setattr(torch.version, "hip", "7.0")
    yield install
    hardware.device_info.cache_clear()
    hardware.detect_arch.cache_clear()


def test_detect_arch_gfx950_is_cdna4(fake_device):
    fake_device("gfx950:sramecc+:xnack-")
    assert hardware.detect_arch() == "cdna4"
    assert hardware.last_level_cache_bytes() == 256 * 1024 * 1024
    assert timer._flush_l2_buffer_mb() == 512


def test_detect_arch_unknown_device(fake_device):
    fake_device("gfx1100")
    assert hardware.detect_arch() is None
    assert hardware.last_level_cache_bytes() == 4 * 1024 * 1024


def test_no_gpu_probes_return_none():
    hardware.device_info.cache_clear()
    hardware.detect_arch.cache_clear()
    if torch.cuda.is_available():
        pytest.skip("host has a GPU")
    assert hardware.device_info() is None and hardware.detect_arch() is None


# ----------------------------------------------------------------------------- metrics


def test_compute_derived_and_roofline():
    cfg = {"flops_expr": "2 * M * K * N", "bytes_expr": "2 * M * K + K * N // 2", "peak_tflops_key": "fp16_mma"}
    res = {"params": {"M": 4096, "K": 4096, "N": 11008}, "dtype": "fp16", "torch_ms": 2.0, "hip_ms": 0.5}
    peak = {"peak_bw_GBs": 8000.0, "peak_tflops": {"fp16_mma": 2500.0}}
    d = metrics.compute_derived(res, cfg, peak)
    tf = 2 * 4096 * 4096 * 11008 / 0.5e-3 / 1e12
    assert d["hip"]["tflops"] == pytest.approx(tf)
    assert d["hip"]["pct_peak_tflops"] == pytest.approx(tf / 2500 * 100)
    assert d["hip"]["speedup"] == pytest.approx(4.0)
    assert "speedup" not in d["torch"]
    # the calibrated peaks (empirical file, "_mma" keys) reported under their own keys
    d = metrics.compute_derived(res, cfg, {"peak_bw_GBs": 8000.0, "peak_tflops": {"fp16": 2500.0}},
                                {"peak_bw_GBs": 6500.0, "peak_tflops": {"fp16_mma": 1950.0}})
    assert d["hip"]["pct_peak_tflops"] == pytest.approx(tf / 2500 * 100)
    assert d["hip"]["pct_calibrated_peak_tflops"] == pytest.approx(tf / 1950 * 100)
    assert d["hip"]["pct_calibrated_peak_bw"] == pytest.approx(d["hip"]["bandwidth_GBs"] / 6500 * 100)
    r = metrics.roofline_pct(1e12, 1e9, 1e-3, 8000.0, 2500.0, bound="mfma")
    assert r["frac"] == pytest.approx(1000 / 2500)
    r = metrics.roofline_pct(0, 8e9, 1e-3, 8000.0, None)
    assert r["bound_by"] == "hbm" and r["frac"] == pytest.approx(1.0)
    # reference rule: the lower ceiling wins (AI = 10 flop/B -> 80 TFLOP/s from HBM)
    r = metrics.roofline_pct(1e11, 1e10, 1e-2, 8000.0, 2500.0)
    assert r["bound_by"] == "hbm" and r["peak"] == pytest.approx(80.0)


def test_config_expressions_evaluate_arithmetic_only():
    ctx = metrics.eval_ctx({"M": 4096, "K": 4096, "N": 11008, "group": 128}, "fp16")
    assert metrics._eval_expr("2 * M * K + K * N // 2 + (K // group) * N * 2", ctx) == \
        2 * 4096 * 4096 + 4096 * 11008 // 2 + 32 * 11008 * 2
    assert metrics._eval_expr("math.ceil(M / 3) + max(K, N) - dtype_size ** 2", ctx) == -(-4096 // 3) + 11008 - 4
    assert metrics._eval_expr("-M % 5", ctx) == (-4096) % 5
    for bad in ("__import__('os')", "M.__class__", "open('x')", "unknown * 2", "M / 0", "[M]", ""):
        assert metrics._eval_expr(bad, ctx) is None, bad
    assert metrics._eval_expr(None, ctx) is None


def test_published_and_calibrated_peak_files():
    pub, cal = metrics.load_peak_config("MI355X"), metrics.load_calibrated_peaks("MI355X")
    assert pub["peak_bw_GBs"] == 8000.0 and pub["peak_tflops"]["fp16"] == 2500.0
    assert pub["peak_tflops"]["fp8_e4m3fn"] == 5000.0
    assert "fp16_mma" in cal["peak_tflops"] and cal["peak_bw_GBs"] < 8000.0
    assert metrics.load_peak_config("no-such-gpu") == {}


# ----------------------------------------------------------------------------- tensors / configs


def test_every_operator_config_expands_and_has_a_generator():
    import yaml

    ops = list_operators()
    assert {"int4_dequant", "w4a16_gemm", "fp8_act_quant", "fp8_scaled_gemm", "moe_topk_gating",
            "moe_w4a16_grouped_gemm"} <= set(ops)
    for op in ops:
        cfg = yaml.safe_load(open(operator_config(op)))
        cases = T.expand_cases(op, cfg)
        assert cases, op
        assert T.get_generator(op) is not None
        assert cfg["benchmark"]["warmup"] == 1 and cfg["benchmark"]["repeat"] == 3  # reference protocol


def test_case_grid_expansion_order_and_expr():
    cases = T._expand_case_grid({"M": {"expr": "[512 * i for i in range(1, 3)]"}, "dtype": ["fp16", "bf16"]},
                                {"K": 8})
    assert cases == [{"K": 8, "M": 512, "dtype": "fp16"}, {"K": 8, "M": 512, "dtype": "bf16"},
                     {"K": 8, "M": 1024, "dtype": "fp16"}, {"K": 8, "M": 1024, "dtype": "bf16"}]
    with pytest.raises(ValueError):
        T._expand_case_grid({"M": []})


def test_generators_are_seeded_and_shaped():
    a = T.generate_int4_dequant_inputs(256, 64, 128, seed=0, device="cpu")
    b = T.generate_int4_dequant_inputs(256, 64, 128, seed=0, device="cpu")
    assert all(torch.equal(x, y) for x, y in zip(a[:3], b[:3]))
    assert a[0].shape == (256, 32) and a[1].shape == (2, 64) and a[2].shape == (2, 32)
    s = a[1].float()
    assert float(s.min()) >= 1e-3 * 0.999 and float(s.max()) <= 1e-2 * 1.001
    (A,) = T.generate_fp8_act_quant_inputs(100, 100, device="cpu")
    big = (A.float().abs() > 6).sum().item()          # the 0.1 % x20 outliers (10 of 10^4)
    assert 5 <= big <= 12
    Aq, Wq, sa, sw = T.generate_fp8_scaled_gemm_inputs(16, 24, 32, device="cpu")
    assert Wq.shape == (32, 24) and Wq.stride() == (1, 32)    # K-contiguous weight operand
    assert sa.shape == (16,) and sw.shape == (24,)


def test_zipf_routing_and_padded_layout():
    choice = T.zipf_routing(2000, 8, 64, s=1.1, seed=4)
    assert choice.shape == (2000, 8)
    assert all(len(set(r.tolist())) == 8 for r in choice)          # distinct experts per token
    counts = torch.bincount(choice.reshape(-1), minlength=64)
    top = counts.sort(descending=True).values
    assert top[0] > 4 * top[-1]                                    # skewed loads
    row_token, offsets, cnt = T.sorted_padded_layout(choice, 64, 128)
    assert offsets[0] == 0 and offsets[-1] == row_token.numel()
    seg = offsets[1:] - offsets[:-1]
    assert (seg % 128 == 0).all() and (seg.long() >= cnt).all()
    for e in (0, 17, 63):
        toks = row_token[offsets[e]:offsets[e] + cnt[e]]
        assert bool((choice[toks] == e).any(dim=1).all())           # every row routed to e
        assert (row_token[offsets[e] + cnt[e]:offsets[e + 1]] == -1).all()


# ----------------------------------------------------------------------------- engine


@pytest.fixture
def fake_operator(monkeypatch, tmp_path):
    """A fake operator `fakeop` with a torch reference and a 'hip' backend module."""
    cfg = tmp_path / "config.yaml"
    cfg.write_text("benchmark: {warmup: 1, repeat: 3}\nverify: {atol: 0, rtol: 0}\ncase_grid:\n  n: [4, 8]\n  dtype: [fp32]\n")
    pkg = "tilebench_amd.benchmarks.operators.fakeop"
    ref = types.ModuleType(pkg + ".impl_torch")
    ref.run = lambda x, n: x * 2
    hip = types.ModuleType(pkg + ".impl_hip")
    calls = []

    def run(x, n):
        calls.append(n)
        return x * 2 if n != 8 else x * 3          # wrong on the second case
    hip.run = run
    hip.get_last_config = lambda: {"tile": 1}
    monkeypatch.setitem(sys.modules, pkg, types.ModuleType(pkg))
    monkeypatch.setitem(sys.modules, pkg + ".impl_torch", ref)
    monkeypatch.setitem(sys.modules, pkg + ".impl_hip", hip)
    monkeypatch.setattr(engine, "operator_config", lambda op: cfg)
    monkeypatch.setattr(engine, "get_generator", lambda op: (lambda n, dtype: (torch.ones(n), n)))
    monkeypatch.setattr(engine, "infer_problem_size", lambda op, p: p["n"])
    monkeypatch.setattr(engine, "HAS_CUDA", True)
    monkeypatch.setattr(engine, "_sync", lambda: None)
    return calls


def test_engine_drives_hip_backend_verifies_and_times(fake_operator):
    timed = []

    def fake_bench(fn, args, kw, **opts):
        timed.append(opts)
        return {"mean": 0.5, "samples": [0.5, 0.5, 0.5]}
    res = engine.run_benchmark_suite("fakeop", enabled_backends=["hip"], bench_fn=fake_bench)
    assert [r["params"]["n"] for r in res] == [4, 8]
    assert res[0]["hip_ok"] and res[0]["hip_ms"] == 0.5 and res[0]["speedup_hip"] == 1.0
    assert not res[1]["hip_ok"] and "bit-exact" in res[1]["hip_err"] and np.isnan(res[1]["hip_ms"])
    assert res[0]["triton_err"].startswith("triton not selected")
    # the torch baseline is timed for both cases, hip only when verified
    assert len(timed) == 3 and timed[0]["warmup"] == 1 and timed[0]["repeat"] == 3


def test_engine_skips_case_when_reference_raises(fake_operator, monkeypatch):
    ref = sys.modules["tilebench_amd.benchmarks.operators.fakeop.impl_torch"]

    def bad(x, n):
        if n == 4:
            raise ValueError("unsupported")
        return x * 2
    monkeypatch.setattr(ref, "run", bad)
    res = engine.run_benchmark_suite("fakeop", enabled_backends=["hip"],
                                     bench_fn=lambda *a, **k: {"mean": 1.0})
    assert [r["params"]["n"] for r in res] == [8]


def test_engine_records_backend_exception(fake_operator):
    hip = sys.modules["tilebench_amd.benchmarks.operators.fakeop.impl_hip"]
    hip.run = lambda x, n: (_ for _ in ()).throw(RuntimeError("tb_x: launch failed"))
    res = engine.run_benchmark_suite("fakeop", enabled_backends=["hip"], bench_fn=lambda *a, **k: {"mean": 1.0})
    assert all(not r["hip_ok"] and "launch failed" in r["hip_err"] for r in res)


def test_engine_missing_backend_module_is_skipped(fake_operator, capsys):
    res = engine.run_benchmark_suite("fakeop", enabled_backends=["hip", "triton"],
                                     bench_fn=lambda *a, **k: {"mean": 1.0})
    assert "triton import skipped" in capsys.readouterr().out
    assert res[0]["triton_err"] == "triton not available"


# ----------------------------------------------------------------------------- timer


def test_kernel_times_are_grouped_per_flushed_sample():
    k = [("tb::fill_kernel(...)", 0.0, 80.0), ("tb::a", 81.0, 5.0), ("tb::b", 87.0, 2.0),
         ("tb::fill_kernel(...)", 100.0, 80.0), ("tb::a", 181.0, 6.0), ("tb::b", 188.0, 2.0)]
    assert timer.kernel_times_per_sample(k, 2, flushed=True) == [0.007, 0.008]
    assert timer.kernel_times_per_sample(k, 3, flushed=True) is None          # wrong sample count
    assert timer.kernel_times_per_sample(k[:4], 2, flushed=True) is None      # a sample without kernels
    assert timer.kernel_times_per_sample([], 1, flushed=True) is None
    plain = [("x", 0.0, 1.0), ("y", 2.0, 3.0), ("x", 6.0, 1.5), ("y", 8.0, 2.5)]
    assert timer.kernel_times_per_sample(plain, 2, flushed=False) == [0.004, 0.004]
    assert timer.kernel_times_per_sample(plain, 3, flushed=False) is None


def test_named_grid_selects_the_reference_gating_grid(fake_operator, tmp_path, monkeypatch):
    cfg = tmp_path / "config.yaml"
    cfg.write_text("benchmark: {warmup: 1, repeat: 3}\nverify: {atol: 0, rtol: 0}\ncase_grid:\n  n: [4]\n"
                   "  dtype: [fp32]\ngrids:\n  wide:\n    case_defaults: {n: 2}\n    case_grid:\n"
                   "      n: [4, 8, 12]\n      dtype: [fp32]\n")
    monkeypatch.setattr(engine, "operator_config", lambda op: cfg)
    res = engine.run_benchmark_suite("fakeop", benchmark_overrides={"grid": "wide"}, enabled_backends=["hip"],
                                     bench_fn=lambda *a, **k: {"mean": 1.0})
    assert [r["params"]["n"] for r in res] == [4, 8, 12]
    with pytest.raises(ValueError, match="no grid named"):
        engine.run_benchmark_suite("fakeop", benchmark_overrides={"grid": "nope"}, enabled_backends=["hip"],
                                   bench_fn=lambda *a, **k: {"mean": 1.0})


def test_gating_config_carries_the_reference_grid():
    import yaml
    cfg = yaml.safe_load(open(operator_config("moe_topk_gating")))
    alt = cfg["grids"]["reference"]
    cases = T.expand_cases("moe_topk_gating", alt)
    assert len(cases) == 60 and {c["dtype"] for c in cases} == {"fp16", "bf16", "fp32"}
    assert {c["E"] for c in cases} == {128} and {c["k"] for c in cases} == {2}
    assert sorted({c["M"] for c in cases}) == [1024 * i for i in range(1, 21)]


def test_reference_device_cpu_runs_the_torch_reference_on_cpu_copies(fake_operator, tmp_path, monkeypatch):
    cfg = tmp_path / "config.yaml"
    cfg.write_text("benchmark: {warmup: 1, repeat: 3}\nverify: {atol: 0, rtol: 0, reference_device: cpu}\n"
                   "case_grid:\n  n: [4]\n  dtype: [fp32]\n")
    monkeypatch.setattr(engine, "operator_config", lambda op: cfg)
    ref = sys.modules["tilebench_amd.benchmarks.operators.fakeop.impl_torch"]
    seen = []
    monkeypatch.setattr(ref, "run", lambda x, n: seen.append(x.device.type) or x * 2)
    res = engine.run_benchmark_suite("fakeop", enabled_backends=["hip"], bench_fn=lambda *a, **k: {"mean": 1.0})
    assert res[0]["hip_ok"] and seen == ["cpu"]
