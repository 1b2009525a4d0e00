"""Profiling support for the hip backend: the kernel manifest of one
impl_hip.run() per operator (probe.py) and validation of a rocprofv3 capture
against it (capture.py), the counterparts of the reference's
scripts/profiling/probe_kernel_count.py and
tilebench/profiling/rocprof_compute.py:100-162."""
