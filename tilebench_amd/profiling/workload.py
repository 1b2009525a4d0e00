"""ONE impl_hip.run() of one case, the program a profiler wraps.

The inputs are generated and the device synchronised first, so a capture
filtered to the backend's kernels (kernels.kernel_filter_regex) holds exactly
the launch sequence of one run(), which capture.validate_capture checks
against the probe's manifest.  Put the interpreter itself after the
profiler's `--`:

    rocprofv3 --kernel-trace --output-format csv -d OUT \\
        --kernel-include-regex '^(?:void )?(?:tb::w4a16::w4a16_decode)' \\
        -- python3 -m tilebench_amd.profiling.workload w4a16_gemm '{"M": 1, "K": 4096, "N": 11008, "group": 128, "dtype": "fp16"}'
"""
from __future__ import annotations

import importlib
import json
import sys

import torch

from tilebench_amd.profiling.probe import _run_kwargs
from tilebench_amd.core.dtypes import resolve_dtype
from tilebench_amd.data.tensors import get_generator


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    if len(argv) != 2:
        print("usage: workload.py OPERATOR CASE_JSON", file=sys.stderr)
        return 2
    op, case = argv[0], json.loads(argv[1])
    impl = importlib.import_module(f"tilebench_amd.benchmarks.operators.{op}.impl_hip")
    params = {k: v for k, v in case.items() if k not in ("dtype", "block_size")}
    inputs = get_generator(op)(**params, dtype=resolve_dtype(case.get("dtype", "fp32")))
    if not isinstance(inputs, tuple):
        inputs = (inputs,)
    torch.cuda.synchronize()
    impl.run(*inputs, **_run_kwargs(impl.run, case))
    torch.cuda.synchronize()
    print(f"workload {op} {json.dumps(case)} done", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
