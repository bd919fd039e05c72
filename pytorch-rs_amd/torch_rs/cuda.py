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
    """Index of the GPU that unindexed "cuda" means (hipGetDevice)."""
    return _C.current_device()


def set_device(device) -> None:
    """Make GPU `device` (an index, or a "cuda:i" device) the current one."""
    if not isinstance(device, int):
        from ._device import parse_device
        d = parse_device("set_device", device)
        if d.type != "cuda" or d.index is None:
            raise ValueError(f"Expected a cuda device with an index, but got: {d}")
        device = d.index
    _C.set_device(device)


def empty_pinned(shape, dtype="float32"):
    """A numpy array (float32 or uint8) in page-locked host memory.  Passing it
    to ``torch_rs.tensor(..., device="cuda")`` or ``copy_to_host`` moves the
    data as one DMA at the PCIe rate; pageable arrays are pipelined through
    the library's own page-locked chunks instead."""
    if isinstance(shape, int):
        shape = (shape,)
    import numpy as np
    return _C.empty_pinned([int(d) for d in shape], np.dtype(dtype).name)


def copy_to_host(tensor, out) -> None:
    """Writes ``tensor``'s logical values into ``out``, a writeable C-contiguous
    float32 array of the same shape, with no intermediate buffer."""
    _C.copy_into(tensor, out)
