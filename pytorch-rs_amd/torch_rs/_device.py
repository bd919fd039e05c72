"""torch_rs.device -- the device descriptor, restated from the reference's
PyDevice (src/python_device.rs:22-385) with the GPU added: the reference
implements only "cpu"; this backend also runs "cuda" (the spelling ROCm
PyTorch uses for an AMD GPU).

Kept exactly: the constructor's argument binding and its errors
(bind_device_constructor, :144-236), device-string validation
(parse_device_string, :81-127), the index rules (an explicit index must be an
int or NumPy integer, non-negative, within int64; every index is narrowed to
a signed byte as PyTorch's DeviceIndex is, :11-15, :269-282), repr (the
narrowed index widened to uint16, :17-20, :329-339), str, hash (the index
byte, :350-352), equality (type and index) and pickling (:354-368).
"""
from __future__ import annotations

import numpy as _np

_UNINDEXED = -1
_TYPES = ("cpu", "cuda")


def _narrow(index: int) -> int:
    """normalize_device_index: the low byte, as a signed 8-bit value."""
    b = index & 0xFF
    return b - 256 if b >= 128 else b


def _constructor_type_name(value) -> str:
    if isinstance(value, device):
        return "torch.device"
    t = type(value)
    return f"numpy.{t.__name__}" if t.__module__ == "numpy" else t.__name__


def _parse_string(function: str, spec: str) -> "device":
    if not spec:
        raise RuntimeError("Device string must not be empty")
    dtype, sep, index = spec.partition(":")
    valid_type = bool(dtype) and all(c.isascii() and (c.isalpha() or c == "_") for c in dtype)
    valid_index = not sep or (bool(index) and all(c in "0123456789" for c in index)
                              and (len(index) == 1 or not index.startswith("0")))
    if not valid_type or not valid_index:
        raise RuntimeError(f"Invalid device string: '{spec}'")
    idx = _UNINDEXED
    if sep:
        value = int(index)
        if value > 2**31 - 1:  # index.parse::<i32>() fails
            raise RuntimeError(f"Could not parse device index '{index}' in device string '{spec}'")
        idx = _narrow(value)
    if dtype not in _TYPES:
        raise RuntimeError(f"{function}(): device '{spec}' is not supported; only 'cpu' and 'cuda' are implemented")
    return device._make(dtype, idx)


def _type_error(function: str, value) -> TypeError:
    argument = "type" if function == "device" else "device"
    return TypeError(f"{function}(): argument '{argument}' must be torch.device or str, not {type(value).__name__}")


def parse_device(function: str, value) -> "device":
    """parse_device_descriptor (src/python_device.rs:67-79): a device, or a
    device string; anything else is a TypeError naming `function`."""
    if isinstance(value, device):
        return value
    if isinstance(value, str):
        return _parse_string(function, value)
    raise _type_error(function, value)


def _check_index_type(index, position):
    if index is None:
        return
    if (isinstance(index, int) and not isinstance(index, bool)) or isinstance(index, _np.integer):
        return
    where = f" (position {position})" if position is not None else ""
    raise TypeError(f"device(): argument 'index'{where} must be int, not {_constructor_type_name(index)}")


def _explicit_index(index) -> int:
    if index is None:
        return _UNINDEXED
    value = int(index)
    if not -(2**63) <= value < 2**63:
        raise ValueError("Overflow when unpacking long long")
    if value < 0:
        raise RuntimeError("Device index must not be negative")
    return _narrow(value)


def _type_and_index(dtype, index, type_position, index_position) -> "device":
    if not isinstance(dtype, str):
        where = f" (position {type_position})" if type_position is not None else ""
        raise TypeError(f"device(): argument 'type'{where} must be str, not {_constructor_type_name(dtype)}")
    _check_index_type(index, index_position)
    parsed = _parse_string("device", dtype)
    if parsed._index != _UNINDEXED:
        raise RuntimeError(
            f"type (string) must not include an index because index was passed explicitly: {dtype}")
    return device._make(parsed._type, _explicit_index(index))


class device:
    """A device descriptor: type "cpu" or "cuda" and an optional index."""

    __slots__ = ("_type", "_index")

    def __new__(cls, *args, **kwargs):
        type_kw = index_kw = device_kw = None
        has_type = has_index = has_device = False
        for key, value in kwargs.items():
            if key == "type":
                type_kw, has_type = value, True
            elif key == "index":
                index_kw, has_index = value, True
            elif key == "device":
                device_kw, has_device = value, True
            else:
                raise TypeError(f"device() got an unexpected keyword argument '{key}'")
        if len(args) == 0:
            if has_type:
                if has_device:
                    raise TypeError("device() got an unexpected keyword argument 'device'")
                return _type_and_index(type_kw, index_kw, None, None)
            if has_device:
                if has_index:
                    raise TypeError('device() missing 1 required positional arguments: "type"')
                return parse_device("device", device_kw)
            raise TypeError(_INVALID)
        if len(args) == 1:
            if has_type:
                raise TypeError("device() got multiple values for argument 'type'")
            if has_device:
                raise TypeError("device() got an unexpected keyword argument 'device'")
            if has_index:
                return _type_and_index(args[0], index_kw, 1, None)
            return parse_device("device", args[0])
        if len(args) == 2 and not (has_type or has_index or has_device):
            return _type_and_index(args[0], args[1], 1, 2)
        raise TypeError(_INVALID)

    @classmethod
    def _make(cls, dtype: str, index: int) -> "device":
        d = object.__new__(cls)
        object.__setattr__(d, "_type", dtype)
        object.__setattr__(d, "_index", index)
        return d

    def __setattr__(self, name, value):
        raise AttributeError(f"'torch_rs.device' object attribute '{name}' is read-only")

    @property
    def type(self) -> str:
        return self._type

    @property
    def index(self):
        return None if self._index == _UNINDEXED else self._index

    def __repr__(self) -> str:
        if self._index == _UNINDEXED:
            return f"device(type='{self._type}')"
        return f"device(type='{self._type}', index={self._index & 0xFFFF})"

    def __str__(self) -> str:
        return self._type if self._index == _UNINDEXED else f"{self._type}:{self._index}"

    def __hash__(self) -> int:
        return self._index & 0xFF

    def __eq__(self, other):
        if not isinstance(other, device):
            return NotImplemented
        return self._type == other._type and self._index == other._index

    def __ne__(self, other):
        eq = self.__eq__(other)
        return eq if eq is NotImplemented else not eq

    def __reduce__(self):
        if self._index == _UNINDEXED:
            return (device, (self._type,))
        return (device, (self._type, self._index))


device.__module__ = "torch_rs"

_INVALID = ("device() received an invalid combination of arguments; expected a device or a type and optional "
            "index")
