"""Correctness check of a backend's outputs against the PyTorch reference.

Same contract as tilebench/core/verifier.py (``_TOLERANCES:4-14``,
``_verify_single:23``, ``verify:44``, ``config_tolerance:59``), extended with
per-output tolerances (a gating result is fp32 weights within 1e-5 plus int32
indices that must match exactly) and a bit-exact mode: atol = rtol = 0 compares
raw bit patterns (fp8 codes, fp16 dequantised values, NaN codes included)
instead of values.
"""
from __future__ import annotations

import torch

_TOLERANCES: dict[torch.dtype, tuple[float, float]] = {
    torch.float32: (1e-5, 1.3e-6),
    torch.float16: (1e-3, 1e-3),
    torch.bfloat16: (1e-2, 1.6e-2),
    torch.float8_e4m3fn: (1.0, 0.1),
    torch.float8_e5m2: (1.0, 0.1),
    torch.int8: (0, 0),
    torch.int16: (0, 0),
    torch.int32: (0, 0),
    torch.int64: (0, 0),
    torch.uint8: (0, 0),
}
_DEFAULT_ATOL = 1e-2
_DEFAULT_RTOL = 1e-2
_FP8_DTYPES = (torch.float8_e4m3fn, torch.float8_e5m2)
_BITS = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}


def _bit_view(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view(_BITS[t.element_size()])


def _verify_single(output: torch.Tensor, reference: torch.Tensor, atol: float | None = None,
                   rtol: float | None = None) -> tuple[bool, str]:
    if not isinstance(output, torch.Tensor):
        return False, f"expected a tensor, got {type(output).__name__}"
    default_atol, default_rtol = _TOLERANCES.get(output.dtype, (_DEFAULT_ATOL, _DEFAULT_RTOL))
    atol = default_atol if atol is None else atol
    rtol = default_rtol if rtol is None else rtol
    if output.shape != reference.shape:
        return False, f"shape mismatch: {tuple(output.shape)} vs {tuple(reference.shape)}"
    if output.dtype != reference.dtype:
        return False, f"dtype mismatch: {output.dtype} vs {reference.dtype}"
    if atol == 0 and rtol == 0:
        o, r = _bit_view(output).cpu(), _bit_view(reference).cpu()
        bad = o != r
        n = int(bad.sum())
        if n == 0:
            return True, ""
        first = tuple(int(i) for i in bad.nonzero()[0])
        return False, (f"bit-exact check failed: {n} of {o.numel()} elements differ; first at {first}: "
                       f"{int(o[first])} vs {int(r[first])}")
    if output.dtype in _FP8_DTYPES:
        output, reference = output.to(torch.float32), reference.to(torch.float32)
    try:
        torch.testing.assert_close(output, reference, atol=atol, rtol=rtol)
        return True, ""
    except Exception as e:  # assert_close raises AssertionError with the mismatch report
        return False, str(e)


def verify(output, reference, atol: float | None = None, rtol: float | None = None,
           per_output=None) -> tuple[bool, str]:
    """Compare a tensor or a tuple of tensors positionally.

    per_output: optional list aligned with the tuple; an entry {atol, rtol}
    replaces the operator-level tolerance for that output, None keeps it."""
    if isinstance(output, (tuple, list)):
        if not isinstance(reference, (tuple, list)) or len(output) != len(reference):
            return False, "output arity differs from the reference"
        for i, (o, r) in enumerate(zip(output, reference)):
            a, t = atol, rtol
            if per_output and i < len(per_output) and per_output[i]:
                a = float(per_output[i].get("atol", a))
                t = float(per_output[i].get("rtol", t))
            ok, err = _verify_single(o, r, atol=a, rtol=t)
            if not ok:
                return False, f"output[{i}]: {err}"
        return True, ""
    return _verify_single(output, reference, atol=atol, rtol=rtol)


def _settings_on(verify_cfg: dict, arch: str | None) -> dict:
    """A config's verify: section with its arch_overrides entry for `arch`
    laid over it (the override wins for every key it names)."""
    merged = dict(verify_cfg)
    merged.update((verify_cfg.get("arch_overrides") or {}).get(arch) or {})
    return merged


def config_tolerance(verify_cfg: dict, arch: str | None) -> tuple[float | None, float | None]:
    """(atol, rtol) of a config's verify: section on `arch`; a value the
    section does not give is None (the output dtype's default then applies)."""
    s = _settings_on(verify_cfg, arch)
    return tuple(None if s.get(k) is None else float(s[k]) for k in ("atol", "rtol"))


def config_per_output(verify_cfg: dict, arch: str | None):
    return _settings_on(verify_cfg, arch).get("per_output")
