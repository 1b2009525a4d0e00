"""The GPU this process runs on: its architecture family and the cache a
cold-entry measurement has to evict.

Interface kept from tilebench/hardware.py (``detect_arch:73``,
``last_level_cache_bytes:95``, the ``_LLC_BYTES:38`` table,
``UncalibratedCacheError``, ``device_info``) because the timer and the
verifier's per-architecture tolerance overrides key on it; the family names are
the reference's ("cdna3", "hopper", "blackwell") plus "cdna4" for gfx950.

The device is looked up once, on first use; importing this module touches no
GPU, and on a host without one every lookup answers None.
"""
from __future__ import annotations

import functools
from typing import NamedTuple

MiB = 1024 * 1024

#: gcnArchName prefix (before the first ':') -> family, for AMD devices.
_AMD_FAMILIES = {"gfx942": "cdna3", "gfx950": "cdna4"}
#: CUDA compute capability -> family, for NVIDIA devices.
_NVIDIA_FAMILIES = {(9, 0): "hopper", (10, 0): "blackwell"}

#: Bytes to evict for a cold-entry measurement on families whose runtime
#: L2_cache_size is not the last-level cache.  On both CDNA families the
#: last level is a 256 MiB Infinity Cache (MALL) behind the per-XCD L2s:
#: cdna3 is the reference's swept MI300X value; cdna4 (MI355X) is registered
#: at the same size, and the flush-size sweep of
#: tilebench_amd/profiling/mall_sweep.py (profiles/mall_sweep_MI355X.txt)
#: shows a 512 MiB flush (the timer's 2x rule) leaves a re-read probe as cold
#: as any larger one.
_LLC_BYTES: dict[str, int] = {"cdna3": 256 * MiB, "cdna4": 256 * MiB}

#: Families whose L2 is known not to be the last level: without an entry in
#: _LLC_BYTES a cold measurement is refused rather than silently warm.
_LLC_CALIBRATION_REQUIRED = frozenset({"cdna3", "cdna4"})


class UncalibratedCacheError(RuntimeError):
    """The eviction size of this architecture's last-level cache is unknown."""


class DeviceInfo(NamedTuple):
    vendor: str                          # "amd" or "nvidia"
    name: str
    capability: tuple[int, int] | None   # NVIDIA only
    gcn_arch_name: str | None            # AMD only, e.g. "gfx950:sramecc+:xnack-"


def _current_properties():
    """(torch, properties of the current device), or None without a GPU."""
    import torch

    if not torch.cuda.is_available():
        return None
    return torch, torch.cuda.get_device_properties(torch.cuda.current_device())


@functools.cache
def device_info() -> DeviceInfo | None:
    try:
        found = _current_properties()
    except Exception:
        return None
    if found is None:
        return None
    torch, props = found
    if torch.version.hip:
        return DeviceInfo("amd", props.name, None, getattr(props, "gcnArchName", None) or None)
    try:
        cap = tuple(torch.cuda.get_device_capability(torch.cuda.current_device()))
    except Exception:
        return None
    return DeviceInfo("nvidia", props.name, cap, None)


@functools.cache
def detect_arch() -> str | None:
    """Family of the current device ("cdna4" for gfx950), or None when there
    is no GPU or the device is outside the families above."""
    info = device_info()
    if info is None:
        return None
    if info.vendor == "amd":
        base = (info.gcn_arch_name or "").partition(":")[0]
        return _AMD_FAMILIES.get(base)
    return _NVIDIA_FAMILIES.get(info.capability)


def last_level_cache_bytes() -> int | None:
    """Bytes a flush must cover to evict the device's last-level cache, or None."""
    family = detect_arch()
    registered = _LLC_BYTES.get(family) if family else None
    if registered is not None:
        return registered
    if family in _LLC_CALIBRATION_REQUIRED:
        raise UncalibratedCacheError(
            f"no validated last-level cache size for {family}: register one in "
            f"tilebench_amd.hardware._LLC_BYTES after an eviction sweep")
    try:
        found = _current_properties()
    except Exception:
        return None
    return None if found is None else found[1].L2_cache_size
