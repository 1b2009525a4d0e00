"""CPU oracle for the ``hip`` backend — TEST INFRASTRUCTURE ONLY.

A plain numpy restatement of what each operator on the hot path computes.  It
is imported only by ``tests/`` and by ``__graft_entry__.smoke()``, always as the
checker.  ``bench.py``'s ``cpu_baseline`` times each operator's torch reference
(``impl_torch.run`` on CPU tensors), not this package.  The shipped backend
(``tilebench_amd``) never imports it and has no CPU fallback.

Reference anchors (Tilebench has no operator for any of these five configs; the
oracle follows the semantics of the nearest reference operators and the
BASELINE config text):

* int4 dequant      — weight_dequant/impl_torch.py:4-8 (elementwise X * S[i//T, j//T],
                      here with int4 codes, zero-points and groups along K);
                      sub-byte unpack as in matmul_int8/impl_torch.py:10-14.
* w4a16 GEMM        — matmul_fp32_fp16_fp8/impl_torch.py:21-27 fp16 path (matmul) on
                      the dequantised weights, fp32 accumulation.
* fp8 act quant     — dequantize_rowwise/impl_torch.py:4-7 (per-row absmax scale)
                      inverted, with torch's float -> float8_e4m3fn cast (RNE, no
                      saturation).
* fp8 scaled GEMM   — matmul_fp32_fp16_fp8/impl_torch.py:10-26 (_scaled_mm, bf16 out)
                      with per-row / per-column scales instead of unit scales.
* block-scaled fp8  — weight_dequant/impl_torch.py:4-8 (X * S[i//T, j//T], T = 128:
                      the 128 x 128 weight-scale map) fused into the fp8 GEMM above,
                      with activations quantised per token and per 128 channels by
                      the fp8 act quant rule applied to each block.
* MoE gating        — moe_topk_gating/impl_torch.py:4-20 (topk, softmax over the k
                      values in fp32, int32 indices) with ties -> lowest index.
* weight_dequant    — weight_dequant/impl_torch.py:4-8; dequantize_rowwise —
                      dequantize_rowwise/impl_torch.py:4-7; quantize_global —
                      quantize_global/impl_torch.py:4-5 (the reference's own operators).
* matmul_int8       — matmul_int8/impl_torch.py:4-19 (2-bit unpack, value - 1, exact).
* matmul_*          — matmul_fp32_fp16_fp8/impl_torch.py:21-27 (matmul; fp8 through
                      a unit-scale _scaled_mm to bf16 and a cast back to e4m3).
* MoE layer         — no reference operator: moe_topk_gating (above), a stable
                      sort of the (token, slot) pairs by expert (the order the
                      config-4 input generator lays rows out in,
                      tilebench_amd/data/tensors.py sorted_padded_layout),
                      the config-4 grouped W4A16 product twice (gate/up with
                      SiLU * up in fp32 between, down scaled by the routing
                      weight) and an in-order fp32 sum over each token's slots.

How each function is pinned (tests/test_oracle.py): closed forms and exact
rational arithmetic (dequant), the torch CPU fp8 cast over every fp16 value and
every e4m3 rounding boundary (fp8 codes), brute-force float64 products on small
inputs and algebraic identities (GEMMs), the reference problem statement's
worked example, a brute-force ranking and float64 softmax (gating).
"""
from .core import (  # noqa: F401
    bf16_bits_to_f32,
    e4m3_from_f32,
    e4m3_to_f32,
    f32_to_bf16_bits,
    fp8_act_quant,
    fp8_act_quant_blocks,
    fp8_block_gemm,
    fp8_scaled_gemm,
    int4_dequant,
    moe_topk_gating,
    moe_w4a16_grouped_gemm,
    pack_int4,
    unpack_int4,
    w4a16_gemm,
    weight_dequant,
    dequantize_rowwise,
    quantize_global,
    unpack_i2,
    matmul_int8,
    matmul_f16,
    matmul_f32,
    matmul_fp8,
    moe_align,
    silu_mul,
    moe_gate_up,
    moe_down,
    moe_combine,
    fused_moe_w4a16,
)
