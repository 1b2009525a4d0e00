"""Package resource locations, resolved from this file (not the CWD).

Mirrors tilebench/paths.py (``OPERATOR_ROOT``, ``PEAK_PERFORMANCE_ROOT``,
``operator_config``) for the resources this package ships.
"""
from __future__ import annotations

import os
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent
DATA_ROOT = PACKAGE_ROOT / "data"
BENCHMARK_ROOT = PACKAGE_ROOT / "benchmarks"
OPERATOR_ROOT = BENCHMARK_ROOT / "operators"
PEAK_PERFORMANCE_ROOT = DATA_ROOT / "peak_performance"
REPO_ROOT = Path(os.environ.get("TILEBENCH_REPO_ROOT") or PACKAGE_ROOT.parent).resolve()
RESULTS_ROOT = REPO_ROOT / "results"


def operator_dir(operator_name: str) -> Path:
    return OPERATOR_ROOT / operator_name


def operator_config(operator_name: str) -> Path:
    path = operator_dir(operator_name) / "config.yaml"
    if not path.is_file():
        raise FileNotFoundError(f"no config.yaml for operator {operator_name!r} at {path}")
    return path


def list_operators() -> list[str]:
    return sorted(p.parent.name for p in OPERATOR_ROOT.glob("*/config.yaml"))
