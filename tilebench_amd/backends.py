"""The backend registry: which implementation modules exist, in which order
results list them, and how a ``--tile-language`` selection is read.

Interface kept from tilebench/backends.py:13-47 so that a selection, a CSV
column order or a result file name means the same thing on both sides:
``BACKEND_ORDER``, ``GPU_BACKENDS``, ``MODES``, ``canonical_backends``,
``parse_backends`` and ``backend_tag``.  The registry below is one table; the
tuples and the parser are derived from it.  ``hip`` (this package's MI355X
kernels) is the last entry.  torch is the baseline every case runs anyway, so it
is accepted in a selection and dropped from it.  This package ships ``impl_hip``
modules only; the other names still parse, and the engine skips a backend whose
module is absent (tilebench/core/engine.py:135-139 does the same for a missing
DSL).
"""
from __future__ import annotations

from typing import Iterable, NamedTuple


class _Entry(NamedTuple):
    name: str
    on_gpu: bool   # measured on the GPU: part of the default selection


_REGISTRY = (
    _Entry("triton", True),
    _Entry("cutile", True),
    _Entry("tilelang", True),
    _Entry("nki", False),      # AWS Trainium: selected only by name
    _Entry("hip", True),       # this package: hand-written gfx950 kernels
)

BACKEND_ORDER = tuple(e.name for e in _REGISTRY)
GPU_BACKENDS = tuple(e.name for e in _REGISTRY if e.on_gpu)
MODES = ("default", "autotune")

_RANK = {name: i for i, name in enumerate(BACKEND_ORDER)}


def canonical_backends(backends: Iterable[str]) -> list[str]:
    """Registry-ordered list of the named backends, each once; a name outside
    the registry is a ValueError."""
    names = set(backends)
    bad = names.difference(_RANK)
    if bad:
        raise ValueError(f"unknown backend(s) {sorted(bad)}; choose from {', '.join(BACKEND_ORDER)}")
    return sorted(names, key=_RANK.__getitem__)


def parse_backends(text: str | None) -> list[str]:
    """Read a comma-separated ``--tile-language`` value (case-insensitive).
    Missing, or containing ``all``: every GPU backend.  ``torch`` is dropped."""
    if text is None:
        return list(GPU_BACKENDS)
    words = {w.strip().lower() for w in text.split(",")} - {""}
    if "all" in words:
        return list(GPU_BACKENDS)
    words.discard("torch")
    return canonical_backends(words)


def backend_tag(backends: Iterable[str]) -> str:
    """Name fragment for result files: the selection joined by '-' in registry
    order (so any typing order gives one tag), or ``torch`` when empty."""
    chosen = canonical_backends(backends)
    return "-".join(chosen) if chosen else "torch"
