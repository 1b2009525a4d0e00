"""The hip backend's launch manifest and a rocprofv3 capture of it.

The probe (torch.profiler) must see exactly the backend's own kernels per
impl_hip.run(), chosen by shape as the C ABI documents; a rocprofv3 kernel
trace of one run, filtered to those kernels, must validate against the probe's
sequence, as the reference checks its captures (rocprof_compute.py:139-162).
"""
import json
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest
import yaml

from tilebench_amd.data.tensors import expand_cases
from tilebench_amd.paths import list_operators, operator_config
from tilebench_amd.profiling import capture as cp
from tilebench_amd.profiling import kernels as kn
from tilebench_amd.profiling import probe

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parent.parent


def _say(*a):
    print("[gpu case]", *a, flush=True)


def _impl(op):
    import importlib
    return importlib.import_module(f"tilebench_amd.benchmarks.operators.{op}.impl_hip")


def _same_after_preparation(r):
    """The first call launched the steady sequence (no operator builds
    per-weight state on its first call)."""
    return r["first_call_identical"]


CASES = [
    ("w4a16_gemm", {"M": 4096, "K": 4096, "N": 11008, "group": 128, "dtype": "fp16"},
     [r"tb::w4a16::w4a16_prefill"]),
    ("w4a16_gemm", {"M": 1, "K": 4096, "N": 11008, "group": 128, "dtype": "fp16"},
     [r"tb::w4a16::w4a16_decode<(false|true)>"]),
    ("w4a16_gemm", {"M": 1, "K": 4096, "N": 11008, "group": 128, "layout": "slabs", "dtype": "fp16"},
     [r"tb::slabs::slab_decode<8, 4>"]),
    ("w4a16_gemm", {"M": 16, "K": 4096, "N": 11000, "group": 128, "dtype": "fp16"},
     [r"tb::w4a16::w4a16_decode<(false|true)>"]),
    ("matmul_int8", {"M": 1024, "N": 1024, "K": 1024, "dtype": "int8"},
     [r"tb::ntg::unpack_i2_tile", r"tb::ntg::nt_gemm<3, 4, \d+, \d+, \d+, \d+>"]),
    ("matmul_fp32_fp16_fp8", {"M": 2048, "N": 2048, "K": 2048, "dtype": "fp16"},
     [r"tb::ntg::transpose_tile<2>", r"tb::ntg::nt_gemm<1, 2, \d+, \d+, \d+, \d+>"]),
    ("matmul_fp32_fp16_fp8", {"M": 1024, "N": 1024, "K": 1024, "dtype": "fp32"},
     [r"tb::ntg::split_rows", r"tb::ntg::split_transpose", r"tb::ntg::nt_gemm<2, 3, \d+, \d+, \d+, \d+>"]),
    ("fp8_act_quant", {"M": 256, "K": 4096, "dtype": "fp16"}, [r"tb::fp8_quant_rows<\d+>"]),
    ("moe_topk_gating", {"M": 1024, "E": 64, "k": 8, "dtype": "fp32"}, [r"tb::filter_kernel<0, 4, 8, 1, true>"]),
    ("moe_topk_gating", {"M": 1024, "E": 128, "k": 2, "dtype": "fp16"}, [r"tb::gating_kernel<1, 16, 8, 2>"]),
]


@pytest.mark.parametrize("op,case,expected", CASES, ids=lambda x: x if isinstance(x, str) else None)
def test_probe_sees_the_kernels_the_shape_selects(gpu, op, case, expected):
    _say("probe", op, case)
    r = probe.probe_case(_impl(op), op, case)
    assert r["count"] == len(expected), r["names"]
    for name, pat in zip(r["names"], expected):
        assert re.fullmatch(pat, name), (name, pat)
    assert r["excluded"] == [], r["excluded"]       # run() itself launches nothing but tb:: kernels
    assert _same_after_preparation(r)


@pytest.mark.parametrize("op", list_operators())
def test_every_operator_launches_only_backend_kernels(gpu, op):
    """Smallest case of each dtype of every grid: one or more tb:: kernels,
    nothing else in a steady-state call, the same sequence on the first call."""
    cfg = yaml.safe_load(open(operator_config(op)))
    cases = expand_cases(op, cfg)
    from tilebench_amd.data.tensors import infer_problem_size
    for dt in sorted({str(c.get("dtype", "fp32")) for c in cases}):
        case = min((c for c in cases if str(c.get("dtype", "fp32")) == dt), key=lambda c: infer_problem_size(op, c))
        _say("probe", op, case)
        r = probe.probe_case(_impl(op), op, case)
        assert r["count"] >= 1 and all(kn.is_backend_kernel(n) for n in r["names"]), r
        assert r["excluded"] == [], r["excluded"]
        assert _same_after_preparation(r), r


def _rocprof(tmp_path, op, case, mode_args, tag):
    out = tmp_path / tag
    cmd = ["timeout", "-s", "KILL", "90", "rocprofv3", *mode_args, "--output-format", "csv",
           "-d", str(out), "-o", "run",
           "--", sys.executable, "-m", "tilebench_amd.profiling.workload", op, json.dumps(case)]
    env = dict(os.environ, TMPDIR=str(tmp_path), PYTHONPATH=str(ROOT))
    res = subprocess.run(cmd, cwd=str(tmp_path), env=env, capture_output=True, text=True, timeout=150)
    assert res.returncode == 0 and "done" in res.stdout, (res.stdout[-2000:], res.stderr[-2000:])
    return out


CAPTURE_CASES = [
    ("matmul_int8", {"M": 1024, "N": 1024, "K": 1024, "dtype": "int8"}),
    ("w4a16_gemm", {"M": 16, "K": 4096, "N": 11008, "group": 128, "dtype": "fp16"}),
    ("matmul_fp32_fp16_fp8", {"M": 512, "N": 512, "K": 512, "dtype": "fp32"}),
]


@pytest.mark.skipif(shutil.which("rocprofv3") is None, reason="rocprofv3 not on PATH")
@pytest.mark.parametrize("op,case", CAPTURE_CASES)
def test_filtered_counter_capture_of_one_run_validates_against_the_probe(gpu, tmp_path, op, case):
    """A counter pass filtered to the manifest's kernels (the form of every
    pass of the reference's counter workloads) holds exactly one run."""
    _say("rocprofv3 --pmc capture", op, case)
    names = probe.probe_case(_impl(op), op, case)["names"]
    out = _rocprof(tmp_path, op, case, ["--pmc", "SQ_WAVES", "--kernel-include-regex",
                                        kn.kernel_filter_regex(names)], "pmc")
    files = sorted(out.rglob("*counter_collection.csv"))
    assert files, list(out.rglob("*"))
    v = cp.validate_capture(files, names)
    assert v["ok"], v


@pytest.mark.skipif(shutil.which("rocprofv3") is None, reason="rocprofv3 not on PATH")
@pytest.mark.parametrize("op,case", CAPTURE_CASES[:2])
def test_kernel_trace_holds_the_probed_backend_launches(gpu, tmp_path, op, case):
    """The unfiltered kernel trace of the workload process (input generation
    and first-call set-up included) holds the probe's backend launches, in
    order, and no other tb:: kernel."""
    _say("rocprofv3 --kernel-trace capture", op, case)
    names = probe.probe_case(_impl(op), op, case)["first_call_names"]  # the workload's run() is a first call
    out = _rocprof(tmp_path, op, case, ["--kernel-trace"], "kt")
    files = sorted(out.rglob("*kernel_trace.csv"))
    assert files, list(out.rglob("*"))
    seq = cp.dispatch_sequence(files[0])
    assert [kn.kernel_stem(n) for n in seq if kn.is_backend_kernel(n)] == names, seq
