"""torch_rs.autograd -- single-root backward (python/torch_rs/autograd/__init__.py:44-127)."""
from __future__ import annotations


def backward(tensors, grad_tensors=None) -> None:
    if isinstance(tensors, (list, tuple)):
        if len(tensors) != 1:
            raise NotImplementedError("torch_rs.autograd.backward supports a single root tensor")
        tensors = tensors[0]
    if grad_tensors is not None:
        raise NotImplementedError("torch_rs.autograd.backward does not support grad_tensors")
    tensors.backward()
