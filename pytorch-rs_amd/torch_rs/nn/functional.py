"""torch_rs.nn.functional -- relu and dropout (python/torch_rs/nn/functional.py:108-143,
src/python_nn_functional.rs:117-200)."""
from __future__ import annotations

import math

import numpy as _np

from .._native import native as _C


def relu(input, inplace: bool = False):
    if inplace:
        raise NotImplementedError("torch_rs.nn.functional.relu does not support inplace=True")
    return input.relu()


def _autograd_suffix(t) -> str:
    name = t._grad_fn_name
    if name is not None:
        return f", grad_fn=<{name}>"
    return ", requires_grad=True" if t.requires_grad else ""


def _format_single_element(t, value: float) -> str:
    """A one-element tensor as PyTorch prints it in this diagnostic
    (python/torch_rs/_diagnostics.py:9-43): integral values as `2.`, others
    with 4 decimals, scientific outside [1e-4, 1e8]; one bracket per dim."""
    finite = math.isfinite(value)
    if finite and value != 0.0:
        integral = value == math.ceil(value)
        scientific = abs(value) > 1.0e8 or abs(value) < 1.0e-4
    else:
        integral, scientific = True, False
    if scientific:
        text = f"{value:.4e}"
    elif integral:
        text = f"{value:.0f}" + ("." if finite else "")
    else:
        text = f"{value:.4f}"
    for _ in range(len(t.shape)):
        text = f"[{text}]"
    return f"tensor({text}{_autograd_suffix(t)})"


def _validate_probability(p):
    """_validate_dropout_probability (python/torch_rs/nn/functional.py:14-24, 86-105)."""
    shown = p
    if isinstance(p, _C.Tensor):
        n = p.numel()
        if n == 0:
            raise RuntimeError("Boolean value of Tensor with no values is ambiguous")
        if n != 1:
            raise RuntimeError("Boolean value of Tensor with more than one value is ambiguous")
        value = p.item()
        shown = value if len(p.shape) == 0 else _format_single_element(p, value)
        p = value
    if p < 0.0 or p > 1.0:
        raise ValueError(f"dropout probability has to be between 0 and 1, but got {shown}")


def _type_name(x) -> str:
    t = type(x)
    return t.__name__ if t.__module__ == "builtins" else f"{t.__module__}.{t.__name__}"


def dropout(input, p: float = 0.5, training: bool = True, inplace: bool = False, *, mask=None):
    """The reference's dropout (python/torch_rs/nn/functional.py:14-31 and the
    bridge src/python_nn_functional.rs:103-200): identity when not training,
    p == 0 or the input is empty; ``input * 0.0`` for p == 1; anything else
    needs sampling, which the reference does not support.  Argument checks
    run in the reference's order with its messages.

    ``mask`` (this backend's addition) is a precomputed keep-mask -- a uint8
    array (or a device byte buffer from ``keep_mask``) of the input's shape
    with 1 = keep -- applied as ``(input * mask) * f32(1/(1-p))``, the
    reference composition ``mul`` then ``mul_scalar``, with the mask read as
    one byte per element."""
    _validate_probability(p)
    op = "dropout_" if inplace else "dropout"
    if not isinstance(input, _C.Tensor):
        raise TypeError(f"{op}(): argument 'input' (position 1) must be Tensor, not {_type_name(input)}")
    prob = float(p.item() if isinstance(p, _C.Tensor) else p)
    if type(training) is not bool:
        raise TypeError(f"{op}(): argument 'train' (position 3) must be bool, not {_type_name(training)}")
    if not 0.0 <= prob <= 1.0:
        if math.isnan(prob):
            shown = "-nan" if math.copysign(1.0, prob) < 0 else "nan"
        else:
            shown = format(prob, ".6g")
        raise RuntimeError(f"dropout probability has to be between 0 and 1, but got {shown}")
    if not training or prob == 0.0 or input.numel() == 0:
        return input
    if mask is not None:
        if inplace:
            raise NotImplementedError("torch_rs.nn.functional.dropout does not support inplace=True")
        if not isinstance(mask, _C.ByteBuffer):
            mask = keep_mask(mask, input.device)
        return _C.mask_apply(input, mask, _np.float32(1.0 / (1.0 - prob)) if prob < 1.0 else _np.float32(0.0))
    if not inplace and prob == 1.0:
        return input * 0.0
    raise NotImplementedError("torch_rs.nn.functional.dropout does not support sampling")


def keep_mask(mask, device="cuda"):
    """Upload a uint8 keep-mask (1 = keep) to the device once, for reuse across steps."""
    arr = _np.asarray(mask, dtype=_np.uint8, order="C")
    return _C.bytes_from_numpy(arr, str(device))
