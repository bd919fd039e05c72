"""torch_rs.accelerator -- accelerator discovery (python/torch_rs/accelerator/__init__.py:1-89).

The reference routes its three public queries through one probe,
``_discover_accelerator()``, which its CPU-only build answers with
(None, False, 0).  This backend answers with the GPU it is built for:
``device("cuda")`` (the device type ROCm PyTorch uses for AMD GPUs), whether
a device is visible now, and how many (hipGetDeviceCount through
libtrs_hip.so).  The queries keep their contracts: ``current_accelerator``
returns the build's accelerator, or None when ``check_available`` is set and
no device is visible.
"""
from __future__ import annotations

from ._device import device as _device
from ._native import native as _C

__all__ = [
    "current_accelerator",
    "device_count",
    "is_available",
]


def _discover_accelerator() -> tuple[_device | None, bool, int]:
    """This backend's accelerator, its availability and the device count."""
    count = _C.device_count()
    return _device("cuda"), count > 0, count


def device_count() -> int:
    """The number of visible accelerator devices (0 when none)."""
    _, _, count = _discover_accelerator()
    return count


def is_available() -> bool:
    """True when at least one accelerator device is visible."""
    _, available, _ = _discover_accelerator()
    return available


def current_accelerator(check_available: bool = False) -> _device | None:
    """The accelerator this backend is built for, as a device with no index;
    None when ``check_available`` is set and no device is visible."""
    accelerator, available, _ = _discover_accelerator()
    if accelerator is not None and ((not check_available) or available):
        return accelerator
    return None
