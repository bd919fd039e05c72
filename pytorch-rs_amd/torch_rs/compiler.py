"""torch_rs.compiler -- the reference's eager compatibility surface for the
torch.compile namespace (python/torch_rs/compiler/__init__.py:1-132,
README.md:178).  Nothing is compiled here: the queries report an eager
program, the default-backend setting is stored process-wide and returned as
given, and assume_constant_result only marks the function.  This backend's
own compilation path is torch_rs.fuse (pointwise programs compiled with
hipRTC)."""
from __future__ import annotations

from collections.abc import Callable
from typing import Any

from . import _compiler_state as _state

__all__ = [
    "assume_constant_result",
    "reset",
    "set_default_backend",
    "get_default_backend",
    "is_compiling",
    "is_dynamo_compiling",
    "is_exporting",
]


def assume_constant_result(fn):
    """Mark `fn` as returning a constant (sets `fn._dynamo_marked_constant` to
    True) and return the same object, unwrapped."""
    fn._dynamo_marked_constant = True
    return fn


def reset() -> None:
    """No compilation caches exist in this eager implementation: does nothing."""
    return None


def set_default_backend(backend: str | Callable[..., Any] | None) -> None:
    """Store the default backend name or callable; None restores "inductor"."""
    if backend is None:
        _state.default_backend = "inductor"
        return
    if not isinstance(backend, str) and not callable(backend):
        raise TypeError(f"backend must be a string or callable, got {type(backend)}")
    _state.default_backend = backend


def get_default_backend() -> str | Callable[..., Any]:
    """The stored default backend (the exact object last set)."""
    return _state.default_backend


def is_compiling() -> bool:
    """False: programs run eagerly."""
    return False


def is_dynamo_compiling() -> bool:
    """False: programs run eagerly."""
    return False


def is_exporting() -> bool:
    """False: nothing is exported."""
    return False
