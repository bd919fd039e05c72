"""torch_rs.cuda -- device queries for the HIP backend (ROCm spells the GPU
device "cuda", as ROCm PyTorch does)."""
from __future__ import annotations

from ._native import native as _C


def is_available() -> bool:
    return _C.device_count() > 0


def device_count() -> int:
    return _C.device_count()


def synchronize() -> None:
    _C.synchronize()


def current_device() -> int:
    return 0
