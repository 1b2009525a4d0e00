"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py) still match the oracle and the seeded generators."""
import os

import numpy as np
import torch

import oracle
from tilebench_amd.data import tensors as T

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return dict(np.load(os.path.join(G, name + ".npz")))


def test_int4_dequant_fixture():
    f = load("int4_dequant")
    p, s, z, *_ = T.generate_int4_dequant_inputs(256, 64, 128, seed=100, device="cpu")
    assert np.array_equal(p.numpy(), f["packed"]) and np.array_equal(z.numpy(), f["zeros"])
    out = oracle.int4_dequant(f["packed"], f["scales"], f["zeros"], int(f["group"]))
    assert np.array_equal(out.view(np.uint16), f["out"].view(np.uint16))


def test_gating_fixture():
    f = load("moe_topk_gating")
    w, i = oracle.moe_topk_gating(f["logits"], int(f["k"]))
    assert np.array_equal(i, f["indices"])
    assert np.array_equal(w, f["weights"])
    assert f["indices"][1].tolist() == list(range(0, 16, 2))   # the tie row: even experts, ascending


def test_fp8_quant_fixture():
    f = load("fp8_act_quant")
    c, sa = oracle.fp8_act_quant(f["A"])
    assert np.array_equal(c, f["codes"]) and np.array_equal(sa.view(np.uint32), f["sa"].view(np.uint32))
    assert (f["codes"][0] == 0xFF).all()


def test_gemm_fixtures():
    f = load("fp8_scaled_gemm")
    assert np.array_equal(oracle.fp8_scaled_gemm(f["Aq"], f["Wq"], f["sa"], f["sw"]), f["Y"])
    f = load("w4a16_gemm")
    assert np.array_equal(oracle.w4a16_gemm(f["A"], f["packed"], f["scales"], f["zeros"], int(f["group"])), f["Y"])
    f = load("moe_w4a16_grouped_gemm")
    Y = oracle.moe_w4a16_grouped_gemm(f["A"], f["packed"], f["scales"], f["zeros"], f["offsets"], int(f["group"]))
    assert np.array_equal(Y, f["Y"])


def test_torch_references_agree_with_fixtures():
    """The harness's PyTorch references (impl_torch) reproduce the fixtures too."""
    from tilebench_amd.benchmarks.operators.fp8_act_quant import impl_torch as fq
    from tilebench_amd.benchmarks.operators.int4_dequant import impl_torch as dq
    from tilebench_amd.benchmarks.operators.moe_topk_gating import impl_torch as gt
    from tilebench_amd.benchmarks.operators.moe_w4a16_grouped_gemm import impl_torch as gg

    f = load("int4_dequant")
    out = dq.run(torch.from_numpy(f["packed"]), torch.from_numpy(f["scales"]), torch.from_numpy(f["zeros"]),
                 256, 64, int(f["group"]))
    assert np.array_equal(out.numpy().view(np.uint16), f["out"].view(np.uint16))
    f = load("moe_topk_gating")
    w, i = gt.run(torch.from_numpy(f["logits"]), 64, 64, int(f["k"]))
    assert np.array_equal(i.numpy(), f["indices"])
    np.testing.assert_allclose(w.numpy(), f["weights"], atol=1e-6)
    f = load("fp8_act_quant")
    q, sa = fq.run(torch.from_numpy(f["A"]))
    assert np.array_equal(q.view(torch.uint8).numpy(), f["codes"])
    f = load("moe_w4a16_grouped_gemm")
    Y = gg.run(*(torch.from_numpy(f[k]) for k in ("A", "packed", "scales", "zeros", "offsets")), int(f["group"]))
    np.testing.assert_allclose(Y.numpy().astype(np.float32), f["Y"].astype(np.float32), atol=1e-2, rtol=1e-2)
