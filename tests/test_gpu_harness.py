"""The reference harness path on the GPU: engine.run_benchmark_suite over real
config.yaml grids, with impl_hip and the real timer (core.timer.report_benchmark:
hipGraph capture, a 512 MiB evicting flush before every sample, hipEvents and
the kernels' own timestamps), as tilebench/core/engine.py:347-358 and
tilebench/core/timer.py:208-284 drive a backend."""
import pytest
import torch

from tilebench_amd.core import engine, timer

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu case]", *a, flush=True)


def _check_rows(rows, min_kernel_ms=0.0):
    assert rows
    for r in rows:
        assert r["hip_ok"], (r["params"], r["dtype"], r["hip_err"])
        st = r["hip_stats"]
        assert st["mode"] == "graph" and st["flush_mb"] == 512
        assert st["time_source"] == "kernel timestamps", st
        assert len(st["samples"]) == len(st["event_samples"]) == 3
        # a sample's kernels run inside its event bracket
        assert 0 < st["mean"] <= st["event_mean"] * 1.02, st
        assert st["mean"] >= min_kernel_ms
        assert r["hip_ms"] == st["mean"]
        print(f"[timer] {r['params']} {r['dtype']}: kernel {st['mean'] * 1e3:.2f} us, "
              f"event bracket {st['event_mean'] * 1e3:.2f} us, profiled runs {st['timestamp_attempts']}, samples "
              f"{[round(v * 1e3, 2) for v in st['samples']]}", flush=True)
        assert r["torch_ms"] > 0 and r["torch_stats"]["mode"] in ("graph", "eager")


def test_engine_int4_dequant_config(gpu):
    _say("engine int4_dequant config.yaml")
    rows = engine.run_benchmark_suite("int4_dequant", enabled_backends=["hip"])
    # 42,270,720 bytes can not move in less than 42.27 MB / 8 TB/s = 5.3 us
    _check_rows(rows, min_kernel_ms=42_270_720 / 8e12 * 1e3)
    assert [r["params"]["K"] for r in rows] == [4096]


def test_engine_gating_config(gpu):
    _say("engine moe_topk_gating config.yaml (BASELINE config 3)")
    rows = engine.run_benchmark_suite("moe_topk_gating", enabled_backends=["hip"])
    _check_rows(rows)
    assert sorted(r["params"]["E"] for r in rows) == [64, 256]


def test_engine_gating_reference_grid(gpu):
    """The reference's own grid (M = 1024..20480, E = 128, k = 2, three dtypes),
    selected by name from the operator's config.yaml: every case verifies."""
    _say("engine moe_topk_gating grid=reference (60 cases, 1 sample each)")
    rows = engine.run_benchmark_suite("moe_topk_gating", benchmark_overrides={"grid": "reference", "repeat": 1,
                                                                              "warmup": 0},
                                      enabled_backends=["hip"])
    assert len(rows) == 60
    assert {r["dtype"] for r in rows} == {"fp16", "bf16", "fp32"}
    assert sorted({r["params"]["M"] for r in rows}) == [1024 * i for i in range(1, 21)]
    for r in rows:
        assert r["hip_ok"], (r["params"], r["dtype"], r["hip_err"])
        assert r["params"]["E"] == 128 and r["params"]["k"] == 2


def test_engine_w4a16_config(gpu):
    """BASELINE config 1 (M = 1, 16, 4096): the decode cases' split-K workspace
    is allocated by the eager verification call, then the graph the timer
    captures reuses it."""
    _say("engine w4a16_gemm config.yaml")
    rows = engine.run_benchmark_suite("w4a16_gemm", enabled_backends=["hip"])
    _check_rows(rows)
    assert [r["params"]["M"] for r in rows] == [1, 16, 4096]


def test_timer_sample_grouping_matches_launch_count(gpu):
    """A run() of two kernels: each sample's device time is the sum of both,
    read between two flush kernels."""
    from tilebench_amd import runtime as rt

    _say("timer two-kernel run")
    n = 1 << 22
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    buf = torch.empty(n * 4, dtype=torch.uint8, device="cuda")

    def two():
        rt.call("tb_l2_flush", buf.data_ptr(), 1 << 20, 0, rt.stream_handle())  # not a 2xLLC flush: part of run()
        return x * 2

    st = timer.report_benchmark(two, (), {}, warmup=1, repeat=3)
    # the fill_kernel inside run() would be read as a flush: grouping refuses and the events are used
    assert st["time_source"] == "hipEvents"
    st = timer.report_benchmark(lambda: x * 2 + 1, (), {}, warmup=1, repeat=3)
    assert st["time_source"] == "kernel timestamps" and st["mode"] == "graph"
    assert st["mean"] <= st["event_mean"]


def test_engine_fp8_act_quant_against_the_cpu_reference(gpu):
    """Bit-exact codes and scales against impl_torch evaluated on the CPU
    (config verify.reference_device: cpu)."""
    _say("engine fp8_act_quant config.yaml")
    rows = engine.run_benchmark_suite("fp8_act_quant", enabled_backends=["hip"])
    _check_rows(rows)


def _grid_slices():
    """The reference's own grids of the analog operators, in slices of at most
    20 cases (each slice one test, so that every test ends within a minute)."""
    import yaml
    from tilebench_amd.data.tensors import expand_cases
    from tilebench_amd.paths import operator_config

    out = []
    for op in ("weight_dequant", "dequantize_rowwise", "quantize_global", "matmul_int8", "matmul_fp32_fp16_fp8"):
        n = len(expand_cases(op, yaml.safe_load(open(operator_config(op)))))
        out += [(op, list(range(i, min(i + 20, n))), n) for i in range(0, n, 20)]
    return out


@pytest.mark.parametrize("op,idx,total", _grid_slices(), ids=lambda v: v if isinstance(v, str) else None)
def test_engine_reference_analog_grid(gpu, op, idx, total):
    """Every case of the reference's grid of each analog operator (weight_dequant
    60, dequantize_rowwise 20, quantize_global 20, matmul_int8 20,
    matmul_fp32_fp16_fp8 60) through the engine with impl_hip: each one
    verifies against impl_torch with the config's tolerance and is timed once."""
    _say(f"engine {op} grid cases {idx[0]}..{idx[-1]} of {total} (1 sample each)")
    rows = engine.run_benchmark_suite(op, benchmark_overrides={"repeat": 1, "warmup": 0, "case_indices": idx},
                                      enabled_backends=["hip"])
    assert len(rows) == len(idx)
    for r in rows:
        assert r["hip_ok"], (op, r["params"], r["dtype"], r["hip_err"])
        assert r["hip_ms"] > 0, (op, r["params"])
    print(f"[grid] {op}: {len(rows)} cases verified, hip_ms "
          f"{min(r['hip_ms'] for r in rows) * 1e3:.1f}..{max(r['hip_ms'] for r in rows) * 1e3:.1f} us", flush=True)


def test_engine_w4a16_slab_grid(gpu):
    """config.yaml's "slabs" grid: the decode shapes on weights the generator
    converted to the slab layout, verified against impl_torch and timed."""
    _say("engine w4a16_gemm grid=slabs")
    rows = engine.run_benchmark_suite("w4a16_gemm", benchmark_overrides={"grid": "slabs"}, enabled_backends=["hip"])
    _check_rows(rows)
    assert [r["params"]["M"] for r in rows] == [1, 16]
    assert all(r["params"]["layout"] == "slabs" and r["hip_config"]["kernel"] == "w4a16_slab_decode" for r in rows)
