"""torch_rs.autograd -- single-root backward with the reference's option
checks (python/torch_rs/autograd/__init__.py:22-127)."""
from __future__ import annotations

import operator as _operator

from .._native import native as _C


def _require_default(name, value, *, allow_none):
    if value is None and allow_none:
        return
    if _operator.index(value):
        raise NotImplementedError(f"torch_rs.autograd.backward does not support {name}=True")


def _single_root(tensors):
    if type(tensors) is _C.Tensor:
        return tensors
    if type(tensors) in (tuple, list) and len(tensors) == 1 and type(tensors[0]) is _C.Tensor:
        return tensors[0]
    raise TypeError("torch_rs.autograd.backward only supports an exact native Tensor, "
                    "directly or in an exact one-element tuple or list")


def backward(tensors, grad_tensors=None, retain_graph=None, create_graph=False, grad_variables=None,
             inputs=None) -> None:
    """Reverse pass from one scalar root, in the reference's order of checks."""
    root = _single_root(tensors)
    if grad_tensors is not None:
        raise NotImplementedError("torch_rs.autograd.backward does not support explicit gradients")
    _require_default("retain_graph", retain_graph, allow_none=True)
    _require_default("create_graph", create_graph, allow_none=False)
    if grad_variables is not None:
        raise NotImplementedError("torch_rs.autograd.backward does not support grad_variables")
    if inputs is not None:
        raise NotImplementedError("torch_rs.autograd.backward does not support inputs")
    root.backward()


from . import grad_mode  # noqa: E402
from .grad_mode import no_grad  # noqa: E402

__all__ = ["backward", "grad_mode", "no_grad"]
