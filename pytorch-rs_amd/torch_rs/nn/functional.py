"""Functional interface."""
# torch_rs.nn.functional: relu and the dropout family, as the reference's
# python/torch_rs/nn/functional.py:1-265 and src/python_nn_functional.rs:13-200.
# The module docstring, relu's docstring and signature are the reference's.

import math
import sys as _sys
import warnings

import numpy as _np

from .._native import native as _C


def relu(input: _C.Tensor, inplace: bool = False) -> _C.Tensor:
    if inplace:
        raise NotImplementedError("torch_rs.nn.functional.relu does not support inplace=True")
    return input.relu()


relu.__doc__ = ("relu(input, inplace=False) -> Tensor\n\n"
                "Applies the rectified linear unit function element-wise. See\n"
                ":class:`~torch.nn.ReLU` for more details.\n") if _sys.version_info >= (3, 13) else (
    """relu(input, inplace=False) -> Tensor

    Applies the rectified linear unit function element-wise. See
    :class:`~torch.nn.ReLU` for more details.
    """)


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


# The reference's dropout family (src/python_nn_functional.rs:13-62): public
# name -> (operation, in-place operation, scalar-tensor p allowed, p == 1
# allowed, input ranks allowed or None).
_DROPOUT_KINDS = {
    "dropout": ("dropout", "dropout_", True, True, None),
    "alpha_dropout": ("alpha_dropout", "alpha_dropout_", False, False, None),
    "feature_alpha_dropout": ("feature_alpha_dropout", "feature_alpha_dropout_", True, True, None),
    "dropout1d": ("feature_dropout", "feature_dropout_", True, False, (2, 3)),
    "dropout2d": ("feature_dropout", "feature_dropout_", True, False, (3, 4)),
    "dropout3d": ("feature_dropout", "feature_dropout_", True, True, (5,)),
}


def _float_like(p, op):
    """parse_float_like_argument (src/python_argument_schema.rs:51-89)."""
    if isinstance(p, _C.Tensor):
        if len(p.shape) == 0 and not p.requires_grad:
            return float(p.item())
        raise TypeError(f"{op}(): argument 'p' (position 2) must be float, not Tensor")
    if isinstance(p, (int, float)):
        return float(p)
    if isinstance(p, _np.bool_):
        return 1.0 if p else 0.0
    if isinstance(p, (_np.integer, _np.floating)):
        return float(p)
    raise TypeError(f"{op}(): argument 'p' (position 2) must be float, not {_type_name(p)}")


def _dropout_bridge(kind, input, p, training, inplace, mask=None):
    """_nn_functional_dropout (src/python_nn_functional.rs:117-200): schema
    checks, then identity when not training, p == 0 or the input is empty;
    ``input * 0.0`` for p == 1 where the kind allows it; sampling is
    unsupported."""
    op_name, inplace_name, tensor_p, p_one, ranks = _DROPOUT_KINDS[kind]
    op = inplace_name if inplace else op_name
    if not isinstance(input, _C.Tensor):
        raise TypeError(f"{op}(): argument 'input' (position 1) must be Tensor, not {_type_name(input)}")
    if not tensor_p and isinstance(p, _C.Tensor):
        raise TypeError(f"{op}(): argument 'p' (position 2) must be float, not Tensor")
    prob = _float_like(p, op)
    if type(training) is not bool:
        raise TypeError(f"{op}(): argument 'train' (position 3) must be bool, not {_type_name(training)}")
    if not 0.0 <= prob <= 1.0:
        if math.isnan(prob):
            shown = "-nan" if math.copysign(1.0, prob) < 0 else "nan"
        else:
            shown = format(prob, ".6g")
        raise RuntimeError(f"dropout probability has to be between 0 and 1, but got {shown}")
    rank = len(input.shape)
    if ranks is not None and rank not in ranks:
        allowed = " or ".join(f"rank-{r}" for r in ranks)
        raise NotImplementedError(f"torch_rs.nn.functional.{kind} only supports {allowed} inputs")
    unbatched_1d = kind == "dropout1d" and rank == 2
    if unbatched_1d and inplace:
        raise NotImplementedError(
            "torch_rs.nn.functional.dropout1d does not support inplace=True for rank-2 inputs")
    if not training or prob == 0.0 or input.numel() == 0:
        # PyTorch runs an unbatched input through unsqueeze(0) and squeeze(0),
        # so even the identity returns a new view with a SqueezeBackward1 edge.
        return input._unsqueeze_front().squeeze(0) if unbatched_1d else input
    if mask is not None:
        if inplace:
            raise NotImplementedError(f"torch_rs.nn.functional.{kind} does not support inplace=True")
        if not isinstance(mask, _C.ByteBuffer):
            mask = keep_mask(mask, input.device)
        return _C.mask_apply(input, mask, _np.float32(1.0 / (1.0 - prob)) if prob < 1.0 else _np.float32(0.0))
    if p_one and not inplace and prob == 1.0:
        return input * 0.0
    raise NotImplementedError(f"torch_rs.nn.functional.{kind} does not support sampling")


def dropout(input, p: float = 0.5, training: bool = True, inplace: bool = False, *, mask=None):
    """The reference's dropout (python/torch_rs/nn/functional.py:14-31, 121-143):
    the Python range check, then the native bridge.

    ``mask`` (this backend's addition) is a precomputed keep-mask -- a uint8
    array (or a device byte buffer from ``keep_mask``) of the input's shape
    with 1 = keep -- applied as ``(input * mask) * f32(1/(1-p))``, the
    reference composition ``mul`` then ``mul_scalar``, with the mask read as
    one byte per element."""
    _validate_probability(p)
    return _dropout_bridge("dropout", input, p, training, inplace, mask)


def dropout1d(input, p: float = 0.5, training: bool = True, inplace: bool = False):
    """python/torch_rs/nn/functional.py:34-40, 146-171."""
    _validate_probability(p)
    input.dim()  # the reference validates the input before the bridge
    return _dropout_bridge("dropout1d", input, p, training, inplace)


def dropout2d(input, p: float = 0.5, training: bool = True, inplace: bool = False):
    """python/torch_rs/nn/functional.py:43-60, 174-199."""
    _validate_probability(p)
    if input.dim() == 3:
        warnings.warn(
            "dropout2d: Received a 3D input to dropout2d and assuming that channel-wise 1D dropout behavior is "
            "desired - input is interpreted as shape (N, C, L), where C is the channel dim. This behavior will "
            "change in a future release to interpret the input as one without a batch dimension, i.e. shape "
            "(C, H, W). To maintain the 1D channel-wise dropout behavior, please switch to using dropout1d "
            "instead.", stacklevel=2)
    return _dropout_bridge("dropout2d", input, p, training, inplace)


def dropout3d(input, p: float = 0.5, training: bool = True, inplace: bool = False):
    """python/torch_rs/nn/functional.py:63-69, 202-227."""
    _validate_probability(p)
    input.dim()
    return _dropout_bridge("dropout3d", input, p, training, inplace)


def alpha_dropout(input, p: float = 0.5, training: bool = False, inplace: bool = False):
    """python/torch_rs/nn/functional.py:72-76, 230-245."""
    _validate_probability(p)
    return _dropout_bridge("alpha_dropout", input, p, training, inplace)


def feature_alpha_dropout(input, p: float = 0.5, training: bool = False, inplace: bool = False):
    """python/torch_rs/nn/functional.py:79-87, 248-265."""
    _validate_probability(p)
    return _dropout_bridge("feature_alpha_dropout", input, p, training, inplace)


def keep_mask(mask, device="cuda"):
    """Upload a uint8 keep-mask (1 = keep) to the device once, for reuse across steps."""
    from .. import _device_str
    arr = _np.asarray(mask, dtype=_np.uint8, order="C")
    return _C.bytes_from_numpy(arr, _device_str(device, "keep_mask"))
