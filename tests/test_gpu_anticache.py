"""The reference's fresh-input checks (tilebench/llm/v2/evaluation/anticache.py:
93-134, restated in tilebench_amd.core.anticache) on every hip operator: fresh
inputs, new values written in place into the same tensors, and a repeat on the
same inputs, each against the operator's torch reference under its config's
tolerances, with no input written and no output aliasing an input."""
import itertools

import pytest
import torch
import yaml

from tilebench_amd.core.anticache import CHECKS, numerical_checks
from tilebench_amd.core.dtypes import resolve_dtype
from tilebench_amd.core.verifier import config_per_output, config_tolerance
from tilebench_amd.data import tensors as T
from tilebench_amd.hardware import detect_arch
from tilebench_amd.paths import list_operators, operator_config

pytestmark = pytest.mark.gpu

# one or more cases per operator, small enough for the torch reference on the GPU
CASES = [
    ("int4_dequant", {"K": 512, "N": 1024, "group": 128}),
    ("w4a16_gemm", {"M": 1, "K": 4096, "N": 11008, "group": 128, "dtype": "fp16"}),
    ("w4a16_gemm", {"M": 16, "K": 4096, "N": 11008, "group": 128, "dtype": "fp16"}),
    ("w4a16_gemm", {"M": 1, "K": 4096, "N": 11008, "group": 128, "layout": "slabs", "dtype": "fp16"}),
    ("w4a16_gemm", {"M": 16, "K": 4096, "N": 11008, "group": 128, "layout": "slabs", "dtype": "fp16"}),
    ("w4a16_gemm", {"M": 300, "K": 512, "N": 1024, "group": 128, "dtype": "fp16"}),
    ("fp8_act_quant", {"M": 256, "K": 4096, "dtype": "fp16"}),
    ("fp8_scaled_gemm", {"M": 512, "N": 512, "K": 1024}),
    ("fp8_act_quant_blocks", {"M": 256, "K": 4096, "dtype": "fp16"}),
    ("fp8_block_scaled_gemm", {"M": 512, "N": 384, "K": 1024}),
    ("moe_topk_gating", {"M": 1024, "E": 64, "k": 8, "dtype": "fp32"}),
    ("moe_topk_gating", {"M": 1024, "E": 256, "k": 8, "dtype": "fp32"}),
    ("moe_topk_gating", {"M": 1024, "E": 128, "k": 2, "dtype": "fp16"}),
    ("moe_w4a16_grouped_gemm", {"tokens": 512, "topk": 8, "experts": 16, "K": 512, "N": 384, "group": 128}),
    ("fused_moe_w4a16", {"tokens": 256, "experts": 8, "topk": 2, "H": 512, "I": 256, "group13": 128,
                         "group2": 64}),
    ("weight_dequant", {"M": 1024, "TILE_SIZE": 128, "dtype": "fp16"}),
    ("weight_dequant", {"M": 1000, "TILE_SIZE": 128, "dtype": "fp32"}),
    ("dequantize_rowwise", {"rows": 256, "cols": 1024}),
    ("quantize_global", {"n": 1 << 20, "dtype": "fp32"}),
    ("matmul_int8", {"M": 512, "N": 512, "K": 1024, "dtype": "int8"}),
    ("matmul_fp32_fp16_fp8", {"M": 512, "N": 512, "K": 1024, "dtype": "fp32"}),
    ("matmul_fp32_fp16_fp8", {"M": 512, "N": 512, "K": 1024, "dtype": "fp16"}),
    ("matmul_fp32_fp16_fp8", {"M": 512, "N": 512, "K": 1024, "dtype": "fp8_e4m3fn"}),
]


def test_every_operator_has_a_case():
    assert {op for op, _ in CASES} == set(list_operators())


def _to(x, device):
    return tuple(t.to(device) if isinstance(t, torch.Tensor) else t for t in x)


def _grouped_maker(params, seeds):
    """Config 4's routing (and so A's padded row count and the offsets) fixed by
    one seed; activations and expert weights new on every call."""
    base = T.generate_moe_w4a16_grouped_gemm_inputs(**params, seed=4, device="cpu")
    A0, offsets, group = base[0], base[4], base[5]
    real = A0.abs().sum(dim=1) != 0

    def make():
        g = torch.Generator().manual_seed(next(seeds))
        A = torch.zeros_like(A0)
        A[real] = torch.randn(int(real.sum()), A0.shape[1], generator=g).to(torch.float16)
        w = T.random_int4_weights(params["K"], params["N"], params["group"], g, experts=params["experts"])
        return _to((A, *w, offsets, group), "cuda")
    return make


@pytest.mark.parametrize("op,case", CASES, ids=[f"{op}-{i}" for i, (op, _) in enumerate(CASES)])
def test_fresh_inputs_same_address_and_repeat(gpu, op, case):
    import importlib

    print("[gpu case] anticache", op, case, flush=True)
    impl_hip = importlib.import_module(f"tilebench_amd.benchmarks.operators.{op}.impl_hip")
    impl_torch = importlib.import_module(f"tilebench_amd.benchmarks.operators.{op}.impl_torch")
    cfg = yaml.safe_load(open(operator_config(op)))
    vcfg = cfg.get("verify", {}) or {}
    atol, rtol = config_tolerance(vcfg, detect_arch())
    per_output = config_per_output(vcfg, detect_arch())
    params = {k: v for k, v in case.items() if k != "dtype"}
    dtype = resolve_dtype(case.get("dtype", "fp32"))
    seeds = itertools.count(100)
    if op == "moe_w4a16_grouped_gemm":
        make = _grouped_maker(params, seeds)
    else:
        gen = T.get_generator(op)

        def make():
            x = gen(**params, dtype=dtype, seed=next(seeds), device="cpu")
            return _to(x if isinstance(x, tuple) else (x,), "cuda")

    if str(vcfg.get("reference_device", "")).lower() == "cpu":
        def reference(*xs):
            out = impl_torch.run(*_to(xs, "cpu"))
            return _to(out, "cuda") if isinstance(out, tuple) else out.to("cuda")
    else:
        reference = impl_torch.run
    res = numerical_checks(impl_hip.run, reference, make, atol=atol, rtol=rtol, per_output=per_output)
    for r in res:
        print(f"  {r.name}: {'ok' if r.ok else 'FAILED ' + r.message[:300]}", flush=True)
    assert [r.name for r in res] == list(CHECKS), res[-1].message
    assert all(r.ok for r in res), [r.message for r in res if not r.ok]
