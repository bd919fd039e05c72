"""torch_rs.autograd.grad_mode -- the no_grad context manager and decorator
(python/torch_rs/autograd/grad_mode.py:1-81); the same object as
torch_rs.no_grad."""
from __future__ import annotations


def __getattr__(name):
    # no_grad is defined in the package root, which imports this module while
    # it initialises; resolve it on first use.
    if name == "no_grad":
        from .. import no_grad
        return no_grad
    raise AttributeError(name)


__all__ = ["no_grad"]
