"""Architecture of the GPU this process runs on, and its last-level cache.

Mirrors tilebench/hardware.py (``detect_arch:73``, ``last_level_cache_bytes:95``,
``_LLC_BYTES:38``) with CDNA4 added: gfx950 (MI350X / MI355X) maps to "cdna4".
Nothing touches the GPU at import time; without a GPU every probe returns None.
"""
from __future__ import annotations

import functools
from typing import NamedTuple

_NVIDIA_ARCH = {(10, 0): "blackwell", (9, 0): "hopper"}
_AMD_ARCH = {"gfx942": "cdna3", "gfx950": "cdna4"}

#: Device-level last-level cache to evict for a cold-entry measurement, where the
#: runtime's L2 size is not that cache.  cdna3: the reference's validated MI300X
#: value.  cdna4 (MI355X): 8 XCDs x 4 MiB L2 in front of a 256 MiB Infinity Cache
#: (MALL) shared by all 256 CUs; the eviction sweep that validates this entry is
#: recorded in profiles/llc_eviction_sweep.txt.
_LLC_BYTES: dict[str, int] = {"cdna3": 256 * 1024 * 1024, "cdna4": 256 * 1024 * 1024}

#: Architectures whose runtime L2 is known not to be the last-level cache.
_LLC_CALIBRATION_REQUIRED = frozenset({"cdna3", "cdna4"})


class UncalibratedCacheError(RuntimeError):
    """The eviction size of this architecture's last-level cache is unknown."""


class DeviceInfo(NamedTuple):
    vendor: str
    name: str
    capability: tuple[int, int] | None
    gcn_arch_name: str | None


@functools.cache
def device_info() -> DeviceInfo | None:
    try:
        import torch

        if not torch.cuda.is_available():
            return None
        index = torch.cuda.current_device()
        props = torch.cuda.get_device_properties(index)
        if torch.version.hip:
            return DeviceInfo("amd", props.name, None, getattr(props, "gcnArchName", None) or None)
        return DeviceInfo("nvidia", props.name, tuple(torch.cuda.get_device_capability(index)), None)
    except Exception:
        return None


@functools.cache
def detect_arch() -> str | None:
    """"cdna4" (gfx950), "cdna3" (gfx942), "blackwell", "hopper" or None."""
    dev = device_info()
    if dev is None:
        return None
    if dev.vendor == "nvidia":
        return _NVIDIA_ARCH.get(dev.capability)
    return _AMD_ARCH.get((dev.gcn_arch_name or "").split(":")[0])


def last_level_cache_bytes() -> int | None:
    """Size of the cache a cold-entry measurement must evict, or None."""
    arch = detect_arch()
    if arch in _LLC_BYTES:
        return _LLC_BYTES[arch]
    if arch in _LLC_CALIBRATION_REQUIRED:
        raise UncalibratedCacheError(f"{arch} LLC eviction size has not been calibrated")
    try:
        import torch

        return torch.cuda.get_device_properties(torch.cuda.current_device()).L2_cache_size
    except Exception:
        return None
