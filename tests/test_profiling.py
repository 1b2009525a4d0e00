"""Capture validation and kernel classification for the hip backend's
profiling, the CPU tests of tests/test_rocprof_compute.py:75-171 restated for
rocprofv3's kernel-trace and counter-collection CSVs."""
import csv
import re

import pytest

from tilebench_amd.profiling import capture as cp
from tilebench_amd.profiling import kernels as kn

#: one run of a two-kernel operator that launches its GEMM twice
PIPELINE = ["tb::ntg::unpack_i2_tile", "tb::ntg::nt_gemm<3, 4, 128, 128, 64, 64>",
            "tb::ntg::unpack_i2_tile", "tb::ntg::nt_gemm<3, 4, 128, 128, 64, 64>"]

TRACE_HEADER = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id", "Kernel_Id",
                "Kernel_Name", "Correlation_Id", "Start_Timestamp", "End_Timestamp"]
COUNTER_HEADER = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id",
                  "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size", "Counter_Name", "Counter_Value",
                  "Start_Timestamp", "End_Timestamp"]


def _trace(path, launches, start=1000):
    """A kernel-trace CSV, rows deliberately written out of launch order."""
    rows = [["KERNEL_DISPATCH", "Agent 1", 1, 0, 7, i + 1, 9, n, i + 1, start + 10 * i, start + 10 * i + 5]
            for i, n in enumerate(launches)]
    with open(path, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(TRACE_HEADER)
        w.writerows(rows[::-1])
    return path


def _counters(path, launches, counters=("FETCH_SIZE", "WRITE_SIZE")):
    """A counter-collection CSV: one row per (dispatch, counter)."""
    with open(path, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(COUNTER_HEADER)
        for i, n in enumerate(launches):
            for c in counters:
                w.writerow([i + 1, i + 1, "Agent 1", 1, 1, 1, 4096, 3, n, 256, c, 1.0, 500 + i, 600 + i])
    return path


@pytest.mark.parametrize("name", [
    "at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<float>>",
    "void at::native::elementwise_kernel<128, 2>(int, void)",
    "__amd_rocclr_copyBuffer", "__amd_rocclr_fillBufferAligned", "Memcpy DtoD", "hipMemsetAsync", "",
    "Cijk_Ailk_Bljk_HHS_BH_MT128x128x32", "tbx::fake_kernel", "my_tb::kernel"])
def test_runtime_library_and_aten_kernels_are_not_operator_kernels(name):
    assert kn.is_aux_kernel(name)
    assert not kn.is_backend_kernel(name)


@pytest.mark.parametrize("name", [
    "tb::w4a16::w4a16_prefill", "void tb::w4a16::w4a16_decode(__half const*, unsigned char const*)",
    "tb::ntg::nt_gemm<1, 2, 256, 256, 128, 64>", "tb::gating_kernel<0, 16, 4, 8>", "tb::copy_kernel"])
def test_backend_kernels_are_operator_kernels(name):
    assert kn.is_backend_kernel(name)
    assert not kn.is_aux_kernel(name)


def test_stem_drops_return_type_and_argument_list_but_keeps_template_arguments():
    assert kn.kernel_stem("void tb::ntg::nt_gemm<1, 2, 256, 256, 128, 64>(unsigned char const*, int)") == \
        "tb::ntg::nt_gemm<1, 2, 256, 256, 128, 64>"
    assert kn.kernel_stem("tb::fp8_quant_rows<4>") == "tb::fp8_quant_rows<4>"
    assert kn.kernel_stem("void tb::f<(tb::Kind)1>(float*)") == "tb::f<(tb::Kind)1>"


def test_kernel_filter_is_start_anchored_never_end_anchored_and_escaped():
    rgx = kn.kernel_filter_regex(PIPELINE + ["at::native::fill"])
    assert rgx.startswith("^") and "$" not in rgx
    pat = re.compile(rgx)
    for n in PIPELINE:
        assert pat.match(n) and pat.match("void " + n + "(int*, int)")
    assert not pat.match("tb::ntg::nt_gemm<3, 4, 256, 256, 128, 64>")   # other template arguments
    assert not pat.match("xtb::ntg::unpack_i2_tile")                     # start-anchored
    assert not pat.match("tb::ntgXunpack_i2_tile")                        # `:` and `<` are literal
    with pytest.raises(ValueError):
        kn.kernel_filter_regex(["at::native::fill"])


def test_repeated_launches_are_counted_not_deduplicated(tmp_path):
    f = _trace(tmp_path / "run_kernel_trace.csv", PIPELINE)
    assert cp.dispatch_sequence(f) == PIPELINE
    g = _counters(tmp_path / "run_counter_collection.csv", PIPELINE)
    assert cp.dispatch_sequence(g) == PIPELINE          # two rows per dispatch, counted once
    v = cp.validate_capture([f, g], PIPELINE)
    assert v["ok"] and v["captured_names"] == PIPELINE
    assert set(v["launches_per_file"].values()) == {4}


def test_argument_lists_in_the_capture_do_not_matter(tmp_path):
    f = _trace(tmp_path / "t.csv", ["void " + n + "(int)" for n in PIPELINE])
    assert cp.validate_capture(f, PIPELINE)["ok"]


def test_a_missing_launch_fails_even_when_every_name_is_right(tmp_path):
    f = _trace(tmp_path / "t.csv", PIPELINE)
    g = _counters(tmp_path / "c.csv", PIPELINE[:3])
    v = cp.validate_capture([f, g], PIPELINE)
    assert not v["ok"]
    assert any("c.csv" in p and "dispatch count 3, manifest expects 4" in p for p in v["problems"])


@pytest.mark.parametrize("intruder", ["__amd_rocclr_copyBuffer", "at::native::vectorized_elementwise_kernel<4>"])
def test_a_non_operator_kernel_in_the_capture_fails(tmp_path, intruder):
    f = _trace(tmp_path / "t.csv", PIPELINE[:2] + [intruder] + PIPELINE[2:])
    v = cp.validate_capture(f, PIPELINE)
    assert not v["ok"] and any("non-operator" in p for p in v["problems"])


def test_launch_order_is_checked(tmp_path):
    f = _trace(tmp_path / "t.csv", [PIPELINE[1], PIPELINE[0]] + PIPELINE[2:])
    v = cp.validate_capture(f, PIPELINE)
    assert not v["ok"] and any("out-of-order dispatch #0" in p for p in v["problems"])


def test_an_unexpected_backend_kernel_fails(tmp_path):
    other = ["tb::ntg::unpack_i2_tile", "tb::ntg::nt_gemm<3, 4, 256, 256, 128, 64>"] * 2
    v = cp.validate_capture(_trace(tmp_path / "t.csv", other), PIPELINE)
    assert not v["ok"] and any("outside the manifest" in p for p in v["problems"])


def test_an_empty_or_absent_capture_fails(tmp_path):
    assert cp.sequence_problems(PIPELINE, []) == ["empty capture: no kernel dispatch recorded"]
    v = cp.validate_capture(_trace(tmp_path / "t.csv", []), PIPELINE)
    assert not v["ok"] and any("empty capture" in p for p in v["problems"])
    v = cp.validate_capture(tmp_path / "absent.csv", PIPELINE)
    assert not v["ok"] and any("missing" in p for p in v["problems"])
    assert not cp.validate_capture([], PIPELINE)["ok"]


def test_probe_needs_a_gpu(monkeypatch, capsys):
    import torch
    from tilebench_amd.profiling import probe
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert probe.main(["--ops", "w4a16_gemm"]) == 2
    assert "needs a GPU" in capsys.readouterr().err


@pytest.mark.parametrize("mangled,stem", [
    ("_ZN2tb5w4a1613w4a16_prefillEPKDF16_PKhS2_S4_PDF16_iiiiii", "tb::w4a16::w4a16_prefill"),
    ("_ZN2tb13gating_kernelILi0ELi16ELi16ELi2EEEvPKvPvPilii", "tb::gating_kernel<0, 16, 16, 2>"),
    ("_ZN2tb11copy_kernelEPKDv4_jPS0_l", "tb::copy_kernel"),
    ("_ZN2tb5w4a1612w4a16_decodeILb0EEEvPKDF16_PKhS3_S5_PDF16_PfPiiiiii", "tb::w4a16::w4a16_decode<false>"),
])
def test_mangled_symbols_as_the_profilers_report_them(mangled, stem):
    """torch.profiler names a HIP kernel by its mangled symbol, rocprofv3 by
    the demangled name (or the mangled one when its demangler cannot read
    `DF16_`).  Every spelling classifies and compares alike, and the filter
    regex selects the mangled one too."""
    assert kn.is_backend_kernel(mangled) and not kn.is_aux_kernel(mangled)
    assert kn.kernel_stem(mangled) == stem
    assert cp.sequence_problems([mangled], [stem]) == []
    assert re.match(kn.kernel_filter_regex([stem]), mangled)
    assert kn.demangle("_Znot_a_symbol") == "_Znot_a_symbol"
    assert kn.is_aux_kernel("_ZN2at6native29vectorized_elementwise_kernelILi4ENS0_11FillFunctorIfEEEEviT0_T1_")


def test_every_kernel_of_the_built_library_is_a_backend_kernel():
    """Each tb:: symbol of libtbhip.so (kernel launch stubs carry the kernel's
    mangled name) demangles into the tb:: namespace, so the probe never drops
    one of the backend's launches whatever its argument types."""
    import shutil
    import subprocess
    from pathlib import Path
    lib = Path(__file__).resolve().parent.parent / "tilebench_amd" / "libtbhip.so"
    if not lib.is_file() or shutil.which("nm") is None:
        pytest.skip("libtbhip.so not built")
    out = subprocess.run(["nm", str(lib)], capture_output=True, text=True, check=True).stdout
    syms = sorted({ln.split()[-1] for ln in out.splitlines()
                   if len(ln.split()) == 3 and ln.split()[1] in "Tt" and ln.split()[-1].startswith("_ZN2tb")})
    assert len(syms) > 20
    for s in syms:
        text = kn.demangle(s)
        assert text != s, s                       # every spelling demangles
        if text.startswith(("tb::", "void tb::")):  # kernels return void; templated helpers name their type
            assert kn.is_backend_kernel(s) and kn.kernel_stem(s).startswith("tb::"), text


def test_filter_regex_under_the_cxx_regex_grammar(tmp_path):
    """rocprofv3 compiles its kernel filter with std::regex (ECMAScript):
    check the filter in that grammar itself, on the names rocprofv3 prints."""
    import shutil
    import subprocess
    if shutil.which("g++") is None:
        pytest.skip("no g++")
    src = tmp_path / "rx.cpp"
    src.write_text('#include <regex>\n#include <iostream>\n#include <string>\n'
                   'int main(int c, char** v) {\n'
                   '  std::regex r(v[1], v[2][0] == \'e\' ? std::regex::extended : std::regex::ECMAScript);\n'
                   '  std::string s;\n'
                   '  while (std::getline(std::cin, s)) std::cout << std::regex_search(s, r) << "\\n"; }\n')
    exe = tmp_path / "rx"
    subprocess.run(["g++", "-O0", "-o", str(exe), str(src)], check=True)
    rgx = kn.kernel_filter_regex(PIPELINE + ["tb::w4a16::w4a16_decode"])
    assert "\\ " not in rgx and "(?" not in rgx
    # the signatures rocprofv3 matches in counter collection: `void ` before templates only
    names = ["tb::ntg::unpack_i2_tile(unsigned char const*, signed char*, int, int)",
             "void tb::ntg::nt_gemm<3, 4, 128, 128, 64, 64>(unsigned char const*, unsigned char const*, void*, int)",
             "tb::w4a16::w4a16_decode(_Float16 const*, int)",
             "void tb::ntg::nt_gemm<3, 4, 256, 256, 128, 64>(unsigned char const*, unsigned char const*, void*, int)",
             "tb::w4a16::w4a16_prefill(_Float16 const*, int)",
             "void at::native::vectorized_elementwise_kernel<4>(int)", "__amd_rocclr_copyBuffer",
             "xtb::ntg::unpack_i2_tile(int)",
             # left mangled by rocprofv3 when it cannot demangle `DF16_`
             "_ZN2tb5w4a1612w4a16_decodeEPKDF16_PKhS2_S4_PDF16_PfPiiiiii",
             "_ZN2tb3ntg7nt_gemmILi3ELi4ELi128ELi128ELi64ELi64EEEvPKhS3_Pviii",
             "_ZN2tb3ntg7nt_gemmILi3ELi4ELi256ELi256ELi128ELi64EEEvPKhS3_Pviii",
             "_ZN2tb5w4a1613w4a16_prefillEPKDF16_PKhS2_S4_PDF16_iiiiii"]
    for grammar in ("ecma", "extended"):
        out = subprocess.run([str(exe), rgx, grammar], input="\n".join(names) + "\n", capture_output=True,
                             text=True, check=True).stdout.split()
        assert out == ["1", "1", "1", "0", "0", "0", "0", "0", "1", "1", "0", "0"], grammar


def test_counter_summary_merges_passes_and_scales_traffic(tmp_path):
    """Counters from two passes of one kernel average over the dispatches that
    report each counter; traffic scales FETCH/WRITE so the copy probe reads its
    known 512 MiB."""
    from tilebench_amd.profiling import counters as pc

    hdr = '"Dispatch_Id","Grid_Size","Kernel_Name","Counter_Name","Counter_Value"\n'

    def write(d, rows):
        d.mkdir()
        (d / "run_counter_collection.csv").write_text(hdr + "".join(
            f'{i},{33554432 if "copy" in k else 256},"{k}","{c}",{v}\n' for i, k, c, v in rows))

    write(tmp_path / "a", [(1, "tb::k(int)", "SQ_WAVES", 10), (2, "tb::k(int)", "SQ_WAVES", 30),
                           (1, "tb::k(int)", "GRBM_GUI_ACTIVE", 800), (2, "tb::k(int)", "GRBM_GUI_ACTIVE", 800)])
    write(tmp_path / "b", [(7, "tb::k(int)", "SQ_VALU_MFMA_BUSY_CYCLES", 512)])
    r = pc.per_dispatch([str(tmp_path / "a"), str(tmp_path / "b")])["tb::k"]
    assert r["dispatches"] == 2
    assert r["counters"] == {"GRBM_GUI_ACTIVE": 800, "SQ_VALU_MFMA_BUSY_CYCLES": 512, "SQ_WAVES": 20}
    assert abs(pc.derived(r["counters"])["mfma_utilisation"] - 512 / (100 * 1024)) < 1e-12
    write(tmp_path / "f", [(1, "tb::copy_kernel(char*)", "FETCH_SIZE", 262144), (2, "tb::x(int)", "FETCH_SIZE", 100)])
    write(tmp_path / "w", [(1, "tb::copy_kernel(char*)", "WRITE_SIZE", 524288), (2, "tb::x(int)", "WRITE_SIZE", 10)])
    t = pc.traffic(str(tmp_path / "f"), str(tmp_path / "w"))
    assert t == {"tb::x": {"fetch_bytes": 204800, "write_bytes": 10240, "fetch_factor": 2.0, "write_factor": 1.0}}


def test_suite_trace_splits_workloads_at_fill_blocks(tmp_path):
    """Each workload's segment starts at a block of fill launches; the timed
    average is over the last `steps` launches of its roofline kernel there."""
    import json

    from tilebench_amd.profiling import suite_trace as st

    fill = "void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<long>, at::detail::Array<char*, 1> >(int, at::native::FillFunctor<long>, at::detail::Array<char*, 1>)"
    seq = [(fill, 1), (fill, 1), ("tb::a(int)", 5), ("tb::a(int)", 7), ("tb::a(int)", 9),
           (fill, 1), ("tb::b(int)", 100), ("tb::a(int)", 1000), ("tb::b(int)", 300), ("tb::b(int)", 500)]
    t, rows = 0, []
    for name, dur in seq:
        rows.append(f'"{name}",{t},{t + dur}\n')
        t += dur + 10
    (tmp_path / "bench_kernel_trace.csv").write_text('"Kernel_Name","Start_Timestamp","End_Timestamp"\n' + "".join(rows))
    (tmp_path / "bench_kernel_stats.csv").write_text('"Name","Calls","AverageNs","MinNs","MaxNs"\n'
                                                     '"tb::a(int)",4,255.25,5,1000\n')
    line = {"steps": 2, "config": {"workload": "wa"}, "roofline": {"kernel": "tb::a"}, "ms_per_step": 0.008,
            "suite": {"wb": {"kernel": "tb::b", "ms": 0.4}}}
    (tmp_path / "bench.json").write_text("[bench] wb: 400 us/step\n" + json.dumps(line) + "\n")
    out = st.summarize(str(tmp_path), str(tmp_path / "bench.json")).splitlines()
    assert out[1].split() == ["wa", "(headline)", "tb::a", "3", "0.01", "8.00"]
    assert out[2].split() == ["wb", "tb::b", "3", "0.40", "400.00"]
    assert out[-1].split() == ["tb::a", "4", "0.26", "0.01", "1.00"]
    with pytest.raises(ValueError, match="fill blocks"):
        line["suite"]["wc"] = {"kernel": "tb::c", "ms": 1.0}
        (tmp_path / "bench.json").write_text(json.dumps(line) + "\n")
        st.summarize(str(tmp_path), str(tmp_path / "bench.json"))


def test_traffic_table_averages_each_workloads_own_dispatches(tmp_path):
    """The counter passes split into workloads at the fill blocks; a kernel shared by
    two workloads is averaged per workload, and the copy probe sets the scale."""
    import json

    from tilebench_amd.profiling import counters as pc

    fill = "void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<long>, at::detail::Array<char*, 1> >(int, at::native::FillFunctor<long>, at::detail::Array<char*, 1>)"
    seq = [(fill, 1), ("tb::d(int)", 10), ("tb::d(int)", 30), (fill, 1), ("tb::d(int)", 100),
           (fill, 1), ("tb::copy_kernel(char*)", 0)]
    for counter, copy_kib in (("FETCH_SIZE", 262144), ("WRITE_SIZE", 524288)):
        d = tmp_path / counter
        d.mkdir()
        rows = "".join(f'{i + 1},{33554432 if "copy" in k else 64},"{k}","{counter}",{copy_kib if "copy" in k else v}\n'
                       for i, (k, v) in enumerate(seq))
        (d / "bench_counter_collection.csv").write_text(
            '"Dispatch_Id","Grid_Size","Kernel_Name","Counter_Name","Counter_Value"\n' + rows)
    line = {"steps": 1, "config": {"workload": "a"}, "ms_per_step": 1.0,
            "roofline": {"kernel": "tb::d", "alg_read_bytes": 10240, "alg_write_bytes": 1024},
            "suite": {"b": {"kernel": "tb::d", "ms": 1.0, "alg_read_bytes": 51200, "alg_write_bytes": 2048},
                      "copy": {"kernel": "tb::copy_kernel", "ms": 1.0}}}
    (tmp_path / "bench.json").write_text(json.dumps(line) + "\n")
    rows = pc.workload_table(str(tmp_path / "FETCH_SIZE"), str(tmp_path / "WRITE_SIZE"), str(tmp_path / "bench.json"))
    assert [(r["workload"], r["dispatches"]) for r in rows] == [("a (headline)", 2), ("b", 1), ("copy", 1)]
    assert rows[0]["fetch_bytes"] == 20 * 1024 * 2.0 and rows[0]["write_bytes"] == 20 * 1024
    assert rows[1]["fetch_bytes"] == 100 * 1024 * 2.0
    text = pc.format_table(rows).splitlines()
    assert text[1].split()[-6:] == ["40", "10", "4.00", "20", "1", "20.00"]


def test_clock_probe_needs_a_gpu(monkeypatch, capsys):
    import torch
    from tilebench_amd.profiling import clock
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert clock.main(["--operator", ""]) == 2
    assert "needs a GPU" in capsys.readouterr().err
