"""Build libtbhip.so (all HIP kernels of the ``hip`` backend) for gfx950.

Each ``csrc/*.hip`` file is compiled to an object with hipcc in parallel, then
the objects are linked into ``tilebench_amd/libtbhip.so`` in-tree, next to the
Python code that loads it.  Cross-compiles without a GPU.

    python -m tilebench_amd.build [--jobs N] [--verbose]
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
LIB = PKG / "libtbhip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-pass-failed",
    # Packed fp32 VALU ops are kept out of every kernel (the generated code
    # uses scalar fp32 ops instead).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


#: extra flags for single sources.  fp8_block.hip: its MFMA results feed VALU
#: FMAs every K step, so they are kept in VGPRs (the default puts MFMA results
#: in AGPRs, which costs a v_accvgpr_read per element before each FMA).
FILE_FLAGS = {
    "fp8_block.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libtbhip.so")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every kernel source and link libtbhip.so; returns its path."""
    hipcc = _hipcc()
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with tempfile.TemporaryDirectory(prefix="tbhip_build_") as tmp:
        objs = [Path(tmp) / (s.stem + ".o") for s in srcs]

        def compile_one(pair):
            src, obj = pair
            cmd = [hipcc, *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
            if verbose:
                print(" ".join(cmd), flush=True)
            proc = subprocess.run(cmd, capture_output=True, text=True)
            if proc.returncode != 0:
                raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stderr[-6000:]}")
            if verbose and proc.stderr.strip():
                print(proc.stderr, file=sys.stderr)
            return obj

        with ThreadPoolExecutor(max_workers=jobs) as pool:
            list(pool.map(compile_one, zip(srcs, objs)))
        tmp_lib = LIB.with_suffix(".so.tmp")
        cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp_lib)]
        if verbose:
            print(" ".join(cmd), flush=True)
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"link failed:\n{proc.stderr[-6000:]}")
        os.replace(tmp_lib, LIB)
    return LIB


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    path = build(args.jobs, args.verbose)
    print(f"built {path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
