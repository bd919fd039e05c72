"""torch_rs.nn.functional -- relu and dropout (python/torch_rs/nn/functional.py:108-143,
src/python_nn_functional.rs:117-200)."""
from __future__ import annotations

import numpy as _np

from .._native import native as _C


def relu(input, inplace: bool = False):
    if inplace:
        raise NotImplementedError("torch_rs.nn.functional.relu does not support inplace=True")
    return input.relu()


def dropout(input, p: float = 0.5, training: bool = True, inplace: bool = False, *, mask=None):
    """The reference's dropout bridge: identity when not training, p == 0 or
    the input is empty; ``input * 0.0`` for p == 1; anything else needs
    sampling, which the reference does not support.

    ``mask`` (this backend's addition) is a precomputed keep-mask -- a uint8
    array (or a device byte buffer from ``keep_mask``) of the input's shape
    with 1 = keep -- applied as ``(input * mask) * f32(1/(1-p))``, the
    reference composition ``mul`` then ``mul_scalar``, with the mask read as
    one byte per element."""
    if not isinstance(input, _C.Tensor):
        raise TypeError(f"dropout(): argument 'input' (position 1) must be Tensor, not {type(input).__name__}")
    p = float(p)
    if not 0.0 <= p <= 1.0:
        raise RuntimeError(f"dropout probability has to be between 0 and 1, but got {p}")
    if not training or p == 0.0 or input.numel() == 0:
        return input
    if mask is not None:
        if inplace:
            raise NotImplementedError("torch_rs.nn.functional.dropout does not support inplace=True")
        if not isinstance(mask, _C.ByteBuffer):
            mask = keep_mask(mask, input.device)
        return _C.mask_apply(input, mask, _np.float32(1.0 / (1.0 - p)) if p < 1.0 else _np.float32(0.0))
    if not inplace and p == 1.0:
        return input * 0.0
    raise NotImplementedError("torch_rs.nn.functional.dropout does not support sampling")


def keep_mask(mask, device="cuda"):
    """Upload a uint8 keep-mask (1 = keep) to the device once, for reuse across steps."""
    arr = _np.asarray(mask, dtype=_np.uint8, order="C")
    return _C.bytes_from_numpy(arr, str(device))
