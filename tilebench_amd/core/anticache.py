"""Fresh-input checks of a backend's run(): a result must come from the
inputs of THIS call.

The reference evaluates a candidate three times in a row
(tilebench/llm/v2/evaluation/anticache.py:93-134, run_numerical_checks):

1. ``fresh_storage``: newly generated inputs (new values at new addresses);
2. ``same_address_new_values``: other values written into the tensors of
   check 1 (same objects, same addresses), which catches a result kept per
   tensor identity or per address;
3. ``repeat_same_inputs``: those inputs once more, which catches state carried
   from one call into the next and inputs corrupted by the previous call.

Each evaluation compares the candidate with the reference under the
operator's tolerances and also fails when the candidate wrote into an input
not declared mutable, or returned an output that shares storage with an input.
The checks stop at the first failure, as there.  This is a restatement of
that protocol, not of its code: the reference output is taken from a private
copy of the inputs (so a reference that writes into its inputs cannot affect
the candidate's call) and mutation is judged on raw bit patterns (NaN inputs
compare equal to themselves).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Iterable

import torch

from tilebench_amd.core.verifier import verify

CHECKS = ("fresh_storage", "same_address_new_values", "repeat_same_inputs")


@dataclass
class CheckResult:
    name: str
    ok: bool
    message: str = ""
    mutated_inputs: list = field(default_factory=list)
    aliased_inputs: list = field(default_factory=list)


def _copy(x):
    """Detached deep copy of the tensors in a (nested) structure."""
    if isinstance(x, torch.Tensor):
        return x.detach().clone()
    if isinstance(x, (tuple, list)):
        return type(x)(_copy(v) for v in x)
    if isinstance(x, dict):
        return {k: _copy(v) for k, v in x.items()}
    return x


def _bits(t: torch.Tensor) -> torch.Tensor:
    t = t.detach().contiguous()
    if t.is_complex() or t.element_size() not in (1, 2, 4, 8):
        return t
    return t.view({1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()])


def _same_bits(a: torch.Tensor, b: torch.Tensor) -> bool:
    return a.shape == b.shape and a.dtype == b.dtype and torch.equal(_bits(a), _bits(b))


def _storage_ids(x) -> set:
    if isinstance(x, torch.Tensor):
        return {x.untyped_storage().data_ptr()} if x.numel() else set()
    if isinstance(x, (tuple, list)):
        out: set = set()
        for v in x:
            out |= _storage_ids(v)
        return out
    if isinstance(x, dict):
        return _storage_ids(list(x.values()))
    return set()


def _write_into(dst: Iterable, src: Iterable) -> None:
    """Copy the tensor values of `src` into the tensors of `dst` in place."""
    for d, s in zip(dst, src):
        if isinstance(d, torch.Tensor):
            if d.shape != s.shape or d.dtype != s.dtype:
                raise ValueError("make_inputs() must return tensors of the same shapes and dtypes every time")
            d.copy_(s)


def _evaluate(name, candidate, reference, inputs, *, atol, rtol, per_output, mutable, sync, allow_aliasing):
    before = _copy(inputs)
    expected = _copy(reference(*_copy(inputs)))
    sync()
    got_raw = candidate(*inputs)
    sync()
    aliased = sorted(i for i, x in enumerate(inputs)
                     if isinstance(x, torch.Tensor) and _storage_ids(x) & _storage_ids(got_raw))
    got = _copy(got_raw)
    mutated = [i for i, (x, b) in enumerate(zip(inputs, before))
               if isinstance(x, torch.Tensor) and not _same_bits(x, b)]
    ok, msg = verify(got, expected, atol=atol, rtol=rtol, per_output=per_output)
    problems = []
    if not ok:
        problems.append(msg)
    stray = [i for i in mutated if i not in mutable]
    if stray:
        problems.append(f"run() wrote into input(s) {stray}, which are read-only")
    if aliased and not allow_aliasing:
        problems.append(f"an output shares storage with input(s) {aliased}; outputs must be fresh")
    _write_into(inputs, before)          # declared-mutable inputs go back to their values
    return CheckResult(name, not problems, "; ".join(problems), mutated, aliased)


def numerical_checks(candidate: Callable, reference: Callable, make_inputs: Callable[[], tuple], *,
                     atol=None, rtol=None, per_output=None, mutable: Iterable[int] = (),
                     sync: Callable[[], None] | None = None, allow_aliasing: bool = False) -> list[CheckResult]:
    """Run the three checks in order; stop after the first that fails.

    make_inputs() returns a new input tuple (new values) on every call, with
    the same shapes and dtypes.  The tolerances and per-output entries are the
    operator's verify settings (core.verifier.verify)."""
    if sync is None:
        sync = torch.cuda.synchronize if torch.cuda.is_available() else (lambda: None)
    opts = dict(atol=atol, rtol=rtol, per_output=per_output, mutable=set(mutable), sync=sync,
                allow_aliasing=allow_aliasing)
    results = []
    inputs = make_inputs()
    for name in CHECKS:
        if name == "same_address_new_values":
            _write_into(inputs, make_inputs())
        results.append(_evaluate(name, candidate, reference, inputs, **opts))
        if not results[-1].ok:
            break
    return results
