"""Backend selection, shared by every entry point.

Same contract as tilebench/backends.py:13-47 (canonical order, ``--tile-language``
parsing, file-name tag) with the MI355X backend ``hip`` appended.  torch is the
implicit baseline and is never part of a selection.  This package ships only
the ``hip`` implementations; the other names stay valid so that a selection
written for the reference parses the same way (their modules are simply absent
here and the engine skips them at import, as the reference does for a missing
DSL, tilebench/core/engine.py:135-139).
"""
from __future__ import annotations

#: Canonical order: drives CSV column order and the backend tag in file names.
BACKEND_ORDER = ("triton", "cutile", "tilelang", "nki", "hip")

#: Backends measured on the GPU itself: the default selection, and what ``all`` means.
GPU_BACKENDS = ("triton", "cutile", "tilelang", "hip")

#: Run modes, as they appear in result file names.
MODES = ("default", "autotune")


def canonical_backends(backends) -> list[str]:
    """The selection as a duplicate-free list in canonical order."""
    chosen = set(backends)
    unknown = sorted(chosen - set(BACKEND_ORDER))
    if unknown:
        raise ValueError(f"unknown backend(s) {unknown}; choose from {', '.join(BACKEND_ORDER)}")
    return [b for b in BACKEND_ORDER if b in chosen]


def parse_backends(text: str | None) -> list[str]:
    """Parse a ``--tile-language`` value. None or ``all`` selects the GPU
    backends; ``torch`` is accepted and ignored because it always runs."""
    if text is None:
        return list(GPU_BACKENDS)
    tokens = [t.strip().lower() for t in text.split(",") if t.strip()]
    if "all" in tokens:
        return list(GPU_BACKENDS)
    return canonical_backends(t for t in tokens if t != "torch")


def backend_tag(backends) -> str:
    """File-name tag of a selection (order-independent); ``torch`` if empty."""
    return "-".join(canonical_backends(backends)) or "torch"
