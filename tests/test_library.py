"""The C-ABI library (no GPU): it loads, exports every entry point that
include/tbhip.h declares, the ctypes table binds all of them, and argument
errors come back as status codes with a message (validation happens on the
host before anything is launched, so these calls touch no device)."""
import ctypes
import os
import re

import pytest

from tilebench_amd import runtime as rt

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tbhip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:tb_status|const char\s*\*)\s+(tb_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    if not rt.LIB_PATH.exists():
        pytest.skip("libtbhip.so is not built (run __graft_entry__.build())")
    return rt.load_library()


def test_header_declares_the_hot_path():
    syms = declared_symbols()
    for s in ("tb_int4_dequant", "tb_w4a16_gemm", "tb_fp8_act_quant", "tb_moe_topk_gating", "tb_version",
              "tb_last_error", "tb_l2_flush"):
        assert s in syms


def test_every_declared_symbol_is_exported_and_bound(lib):
    syms = declared_symbols()
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in tbhip.h but not exported"
    bound = set(rt.SIGNATURES) | set(rt.STRING_SYMBOLS)
    assert set(syms) == bound, f"ctypes table differs from the header: {set(syms) ^ bound}"


def test_version_string(lib):
    assert rt.version().startswith("tbhip ") and "gfx950" in rt.version()


def test_argument_errors_are_statuses_with_messages(lib):
    assert lib.tb_int4_dequant(None, None, None, None, 4, 4, 2, None) == rt.TB_E_INVALID
    assert "null pointer" in lib.tb_last_error().decode()
    fake = 1 << 40  # never dereferenced: shape checks fail first
    assert lib.tb_int4_dequant(fake, fake, fake, fake, 4, 5, 2, None) == rt.TB_E_INVALID
    assert "even" in lib.tb_last_error().decode()
    assert lib.tb_moe_topk_gating(fake, fake, fake, 16, 64, 65, 0, None) == rt.TB_E_INVALID
    assert lib.tb_fp8_act_quant(fake + 4, fake, fake, 4, 16, None) == rt.TB_E_ALIGN
    assert lib.tb_w4a16_gemm(fake, fake, fake, fake, fake, 64, 64, 100, 128, None, 0, None) == rt.TB_E_INVALID
    with pytest.raises(ValueError, match="tb_int4_dequant"):
        rt.check(lib.tb_int4_dequant(None, None, None, None, 4, 4, 2, None), "tb_int4_dequant")


def test_w4a16_workspace_contract(lib):
    need = ctypes.c_int64(-1)
    assert lib.tb_w4a16_workspace_size(4096, 11008, 4096, 128, ctypes.byref(need)) == rt.TB_OK
    assert need.value == 0                                   # prefill: no workspace
    assert lib.tb_w4a16_workspace_size(16, 11008, 4096, 128, ctypes.byref(need)) == rt.TB_OK
    assert need.value > 16 * 11008 * 4                       # decode: counters + split partials
    fake = 1 << 40
    assert lib.tb_w4a16_gemm(fake, fake, fake, fake, fake, 16, 11008, 4096, 128, None, 0, None) == rt.TB_E_INVALID
    assert "workspace" in lib.tb_last_error().decode()


def test_w4a16_refuses_operands_past_2gib(lib):
    """Buffer offsets are 32-bit with a 2^31 out-of-range sentinel: an A, W or
    scale operand of 2 GiB or more is refused before any launch."""
    fake = 1 << 40
    # prefill with M * K * 2 = 2^31 bytes of A
    assert lib.tb_w4a16_gemm(fake, fake, fake, fake, fake, 1 << 18, 11008, 4096, 128, None, 0, None) \
        == rt.TB_E_INVALID
    assert "2 GiB" in lib.tb_last_error().decode()
    # W of K * N / 2 = 2^31 bytes (decode shape)
    assert lib.tb_w4a16_gemm(fake, fake, fake, fake, fake, 1, 1 << 16, 1 << 16, 128, None, 0, None) \
        == rt.TB_E_INVALID
    assert "2 GiB" in lib.tb_last_error().decode()
    # just below the limit the shape checks pass and the missing workspace is what fails
    assert lib.tb_w4a16_gemm(fake, fake, fake, fake, fake, 16, 11008, 4096, 128, None, 0, None) == rt.TB_E_INVALID
    assert "workspace" in lib.tb_last_error().decode()


def test_noalloc_entry_point_checks_before_touching_a_device(lib):
    fake = 1 << 40
    assert lib.tb_w4a16_gemm_noalloc(None, fake, fake, fake, fake, 16, 11008, 4096, 128, None) == rt.TB_E_INVALID
    assert "tb_w4a16_gemm_noalloc: null pointer" in lib.tb_last_error().decode()
    assert lib.tb_w4a16_gemm_noalloc(fake, fake, fake, fake, fake, 1, 1 << 16, 1 << 16, 128, None) \
        == rt.TB_E_INVALID
    assert "2 GiB" in lib.tb_last_error().decode()
    assert lib.tb_w4a16_gemm_noalloc(fake + 8, fake, fake, fake, fake, 4, 64, 64, 64, None) == rt.TB_E_ALIGN


def test_no_device_means_loud_failure():
    import torch

    if torch.cuda.is_available():
        pytest.skip("host has a GPU")
    with pytest.raises(rt.HipBackendUnavailable):
        rt.require_device()
