"""torch_rs -- the pytorch-rs Python API for the MI355X device backend.

Mirrors the hot-path surface of the reference package (python/torch_rs and
the PyO3 module, src/python.rs:10558-10634): ``tensor``, ``relu``, ``exp``,
``matmul``, ``mul``, ``no_grad``, the Tensor arithmetic and view methods,
``backward`` / ``.grad``, ``nn.functional.relu/dropout`` and
``get_float32_matmul_precision() == "highest"``.  Tensors created with
``device="cuda"`` live in HBM and every op runs as a HIP kernel through
libtrs_hip.so; ``"cpu"`` tensors are host staging for ``.to()`` only.

Additions of this backend (absent from the reference, documented where
they differ): device tensors record VJPs for matmul, tensor-tensor add/sub
and exp; ``fuse`` compiles a pointwise function into one hipRTC kernel;
``nn.functional.dropout`` accepts a precomputed uint8 keep-mask; ``device``
and ``accelerator`` know the "cuda" device type besides "cpu".
"""
from __future__ import annotations

import builtins as _builtins
import contextlib
import operator as _operator

import numpy as _np

from ._device import device, parse_device as _parse_device
from ._native import native as _C

Tensor = _C.Tensor
float32 = "torch_rs.float32"
float = float32  # noqa: A001  (the reference exports torch_rs.float too)
__version__ = "0.1.0+mi355x"

def _device_str(device, function: str = "tensor") -> str:
    """The engine's device string for a factory's ``device`` argument: None
    is the CPU, an indexed CPU descriptor is the CPU (the reference keeps CPU
    storage unindexed), an unindexed "cuda" is the current GPU."""
    if device is None:
        return "cpu"
    d = _parse_device(function, device)
    if d.type == "cpu":
        return "cpu"
    index = d.index if d.index is not None else _C.current_device()
    if index < 0:
        raise RuntimeError(f"{function}(): invalid device ordinal {index}")
    return f"cuda:{index}"


def _flatten(data):
    """Nested sequences -> (flat list, shape), rejecting ragged input."""
    if isinstance(data, (int, _builtins.float, _np.integer, _np.floating)):
        return [data], ()
    seq = list(data)
    if not seq:
        return [], (0,)
    parts = [_flatten(x) for x in seq]
    shape0 = parts[0][1]
    for _, s in parts:
        if s != shape0:
            raise ValueError(f"expected sequence of length {shape0[0] if shape0 else 0} at dim 1")
    flat = [v for p, _ in parts for v in p]
    return flat, (len(seq),) + shape0


def _requires_grad_arg(function: str, value, allow_none: bool) -> bool:
    """parse_requires_grad / parse_factory_requires_grad (src/python.rs:4189-4215):
    an exact builtin bool (or None where the factory allows it)."""
    if value is None and allow_none:
        return False
    if type(value) is bool:
        return value
    raise TypeError(f"{function}(): argument 'requires_grad' must be bool, not {_py_type_name(value)}")


def tensor(data, *, dtype=None, device=None, requires_grad=False) -> Tensor:
    """torch_rs.tensor (src/python.rs:4139-4170): float32 values from a
    number, a nested sequence, or any buffer/array (copied, row-major)."""
    requires_grad = _requires_grad_arg("tensor", requires_grad, False)
    if dtype not in (None, float32):
        raise TypeError("torch_rs supports only float32 tensors")
    if isinstance(data, Tensor):
        arr = data.numpy()
    elif isinstance(data, (bytes, bytearray)):
        raise TypeError("new(): invalid data type 'bytes'")
    elif isinstance(data, (memoryview, _np.ndarray)):
        arr = _np.asarray(data, dtype=_np.float32)
    else:
        flat, shape = _flatten(data)
        arr = _np.asarray(flat, dtype=_np.float64).astype(_np.float32).reshape(shape)
    # asarray(order="C") keeps 0-d arrays 0-d (ascontiguousarray would make them [1]).
    t = _C.from_numpy(_np.asarray(arr, dtype=_np.float32, order="C"), _device_str(device, "tensor"))
    return t.with_requires_grad(bool(requires_grad))


def zeros(*shape, device=None, requires_grad=False) -> Tensor:
    return _full("zeros", shape, 0.0, device, requires_grad)


def ones(*shape, device=None, requires_grad=False) -> Tensor:
    return _full("ones", shape, 1.0, device, requires_grad)


def full(shape, fill_value, *, device=None, requires_grad=False) -> Tensor:
    return _full("full", (shape,), fill_value, device, requires_grad)


def _full(function, shape, fill_value, device, requires_grad) -> Tensor:
    """The size is one sequence or int (bind_creation_arguments,
    src/python.rs:4527-4560), or, as in PyTorch, several ints."""
    requires_grad = _requires_grad_arg(function, requires_grad, True)
    if shape and not isinstance(shape[0], int) and len(shape) > 1:
        raise TypeError(f"{function}() takes 1 positional argument but {len(shape)} were given")
    if len(shape) == 1 and not isinstance(shape[0], int):
        shape = tuple(shape[0])
    return _C.full([int(d) for d in shape], _np.float32(fill_value),
                   _device_str(device, function)).with_requires_grad(bool(requires_grad))


def is_tensor(obj) -> bool:
    return isinstance(obj, Tensor)


# ---- variable functions (src/python_variable_functions.rs:32-63) ----------

def relu(input: Tensor) -> Tensor:
    return input.relu()


def _unary_out(name, input, out, autograd_error=None):
    """Top-level unary with the reference's `out` and autograd guards
    (apply_top_level_unary_out, src/python.rs:1784-1820, 2673-2694).  The
    autograd guard applies to host tensors; device tensors record the VJP."""
    if out is not None:
        raise RuntimeError(f"{name}(): the 'out' argument is not supported")
    if (autograd_error and isinstance(input, Tensor) and not input.is_cuda and input.requires_grad
            and is_grad_enabled()):
        raise RuntimeError(autograd_error)


def exp(input: Tensor, *, out=None) -> Tensor:
    _unary_out("exp", input, out, "exp(): autograd recording is not supported")
    return input.exp()


def neg(input: Tensor, *, out=None) -> Tensor:
    _unary_out("neg", input, out)
    return input.neg()


def negative(input: Tensor, *, out=None) -> Tensor:
    _unary_out("negative", input, out)
    return input.neg()


def add(input, other):
    return input + other


def sub(input, other):
    return input - other


def mul(input, other):
    return input * other


multiply = mul


def div(input, other):
    return input / other


def matmul(*args, **kwargs) -> Tensor:
    """torch_rs.matmul(input, other) -- also as matmul(input=, other=) or
    matmul(x1=, x2=), the keyword spellings the reference accepts."""
    left, right = _two_operands("matmul", args, kwargs, (("input", "other"), ("x1", "x2")))
    return left.matmul(right)


def _two_operands(name, args, kwargs, spellings):
    if "out" in kwargs:
        raise TypeError(f"{name}() got an unexpected keyword argument 'out'")
    if len(args) == 2 and not kwargs:
        return args
    for first, second in spellings:
        if len(args) == 1 and set(kwargs) == {second}:
            return args[0], kwargs[second]
        if not args and set(kwargs) == {first, second}:
            return kwargs[first], kwargs[second]
    raise TypeError(f"{name}() received an invalid combination of arguments")


def sum(input: Tensor) -> Tensor:  # noqa: A001
    return input.sum()


def permute(input: Tensor, dims) -> Tensor:
    return input.permute(dims)


def transpose(input: Tensor, dim0: int, dim1: int) -> Tensor:
    return input.transpose(dim0, dim1)


def t(input: Tensor) -> Tensor:
    return input.t()


def clone(input: Tensor) -> Tensor:
    return input.clone()


def get_float32_matmul_precision() -> str:
    """fp32 matmul runs on FP32 MFMA with fp32 accumulation: always "highest"
    (python/torch_rs/__init__.py:81-85)."""
    return "highest"


def set_float32_matmul_precision(precision: str) -> None:
    if precision != "highest":
        raise RuntimeError("torch_rs runs fp32 matmul at 'highest' precision only")


def get_num_threads() -> int:
    return 1


# ---- grad mode (src/grad_mode.rs) ---------------------------------------

class no_grad(contextlib.ContextDecorator):
    """Thread-local no-grad scope, usable as a context manager or decorator."""

    def __enter__(self):
        _C.enter_no_grad()
        return self

    def __exit__(self, *exc):
        _C.exit_no_grad()
        return False


def is_grad_enabled() -> bool:
    return _C.is_grad_enabled()


# ---- Tensor conveniences (src/python.rs:3527-3919) ------------------------

def _stride(self, dim=None):
    s = self._strides()
    if dim is None:
        return s
    r = max(len(s), 1)
    if not -r <= dim < r:
        raise IndexError(f"Dimension out of range (expected to be in range of [-{r}, {r - 1}], but got {dim})")
    return s[dim]


def _size(self, dim=None):
    if dim is None:
        return self.shape
    return self.shape[dim]


class _GradFn:
    """Python-visible backward node (src/autograd_node.rs): named by class."""

    _classes: dict = {}

    @classmethod
    def of(cls, name):
        if name not in cls._classes:
            cls._classes[name] = type(name, (cls,), {})
        return cls._classes[name]()

    def name(self):
        return type(self).__name__

    def __repr__(self):
        return f"<{type(self).__name__} object>"


def _grad_fn(self):
    n = self._grad_fn_name
    return None if n is None else _GradFn.of(n)


def _grad(self):
    """Tensor.grad (src/python_tensor_leaf_grad.rs:50-66): None until a backward
    reaches this leaf, then one cached tensor aliasing the accumulated
    gradient, so a retained `.grad` sees later accumulation in place."""
    key = self._autograd_id()
    cached = self.__dict__.get("_grad_cache")
    if cached is not None and cached[0] == key:
        return cached[1]
    if not self._has_grad():
        return None
    g = self._live_grad()
    self.__dict__["_grad_cache"] = (key, g)
    return g


_EXP_LOW, _EXP_HIGH = _np.float32(1e-4), _np.float32(1e16)


def _rust_f32_debug(v) -> str:
    """One f32 as Rust's `{:?}` prints it: the shortest digits that round-trip,
    in positional form with at least one fractional digit, or in exponent form
    (`1e-5`, `1.5e16`) when 0 < |v| < 1e-4 or |v| >= 1e16; `NaN`, `inf`, `-inf`."""
    v = _np.float32(v)
    if _np.isnan(v):
        return "NaN"
    if _np.isinf(v):
        return "inf" if v > 0 else "-inf"
    a = abs(v)
    if a != 0 and (a < _EXP_LOW or a >= _EXP_HIGH):
        return _np.format_float_scientific(v, unique=True, trim="-", exp_digits=1).replace("e+", "e")
    return _np.format_float_positional(v, unique=True, trim="0")


def _repr(self):
    """`tensor({values:?}, shape={shape:?})`: every logical value in row-major
    order and the shape, as the reference's Tensor.__repr__ (src/python.rs:3933-3942)."""
    values = ", ".join(_rust_f32_debug(v) for v in self.numpy().reshape(-1))
    shape = ", ".join(str(d) for d in self.shape)
    return f"tensor([{values}], shape=[{shape}])"


def _array(self, dtype=None, copy=None):
    """__array__ (src/python.rs:3744-3756, 4031-4052): always a copy of the
    logical values, float32 unless `dtype` is given."""
    if copy is False:
        raise ValueError("cannot create a non-copying NumPy view of tensor storage")
    a = self.numpy()
    return a if dtype is None else a.astype(dtype)


def _bool(self):
    """truth_value (src/python.rs:4015-4029): one element -> value != 0."""
    n = self.numel()
    if n == 0:
        raise RuntimeError("Boolean value of Tensor with no values is ambiguous")
    if n != 1:
        raise RuntimeError("Boolean value of Tensor with more than one value is ambiguous")
    return self.item() != 0.0


def _len(self):
    if not self.shape:
        raise TypeError("len() of a 0-d tensor")
    return self.shape[0]


Tensor.stride = _stride
Tensor.size = _size
Tensor.grad_fn = property(_grad_fn)
Tensor.grad = property(_grad)
Tensor.dtype = property(lambda self: float32)
Tensor.ndim = property(lambda self: self.dim())
_native_to = Tensor.to


def _tensor_device(self) -> device:
    """device(type='cpu') for host tensors, device(type='cuda', index=i) on GPU i."""
    s = self._device_str
    if s == "cpu":
        return device("cpu")
    return device("cuda", int(s.split(":")[1]))


def _to(self, *args, **kwargs):
    """Tensor.to(device): a copy on that device (the same tensor if already there)."""
    if len(args) + len(kwargs) != 1 or (kwargs and "device" not in kwargs):
        raise TypeError("to() supports only a device argument: to(device) or to(device=...)")
    return _native_to(self, _device_str(args[0] if args else kwargs["device"], "to"))


def _cuda(self, device=None):
    """Tensor.cuda(device=None): to the current GPU, or GPU `device` (an index,
    a device or a device string)."""
    if device is None:
        return _native_to(self, f"cuda:{_C.current_device()}")
    if isinstance(device, int) and not isinstance(device, bool):
        return _native_to(self, f"cuda:{device}")
    d = _parse_device("cuda", device)
    if d.type != "cuda":
        raise RuntimeError(f"Invalid device, must be cuda device: {d}")
    return _native_to(self, _device_str(d, "cuda"))


_native_permute = Tensor.permute


def _py_type_name(x) -> str:
    """python_type_name (src/python.rs:9635-9701): "Tensor" / "torch.device"
    for the package's own types, else CPython's tp_name: the bare name for
    classes defined in Python, "module.name" for extension types
    (numpy.bool, numpy.float64)."""
    t = type(x)
    if t is Tensor:
        return "Tensor"
    if t is device:
        return "torch.device"
    if t.__flags__ & (1 << 9) or t.__module__ == "builtins":  # Py_TPFLAGS_HEAPTYPE
        return t.__name__
    return f"{t.__module__}.{t.__name__}"


def _is_dim(x) -> bool:
    if isinstance(x, bool):
        return False
    try:
        _operator.index(x)
        return True
    except TypeError:
        return False


def _permute_dims(args, kwargs) -> list:
    """bind_permute_dimensions / parse_permute_dimensions (src/python.rs:9321-9510):
    permute(*dims), permute(dims) with a tuple or list, or permute(dims=...)."""
    keyword, error = None, None
    for key, value in kwargs.items():
        if key == "dims" and not args and keyword is None:
            keyword = value
        elif key == "dims":
            error = error or TypeError("permute() got multiple values for argument 'dims'")
        else:
            error = error or TypeError(f"permute() got an unexpected keyword argument '{key}'")

    def sequence(value, position):
        where = f" (position {position})" if position is not None else ""
        if not isinstance(value, (tuple, list)):
            raise TypeError(f"permute(): argument 'dims'{where} must be tuple of ints, not {_py_type_name(value)}")
        if value and not _is_dim(value[0]):
            if position is None:
                raise TypeError(f"permute(): argument 'dims' must be tuple of ints, not {_py_type_name(value)}")
            raise TypeError(f"permute(): argument 'dims'{where} must be tuple of ints, but found element of type "
                            f"{_py_type_name(value[0])} at pos 0")
        return list(value)

    if not args:
        if keyword is None:
            raise TypeError('permute() missing 1 required positional arguments: "dims"')
        dims = sequence(keyword, None)
    elif len(args) == 1:
        if isinstance(args[0], (tuple, list)):
            dims = sequence(args[0], 1)
        elif _is_dim(args[0]):
            dims = list(args)
        else:
            raise TypeError(f"permute(): argument 'dims' (position 1) must be tuple of ints, not "
                            f"{_py_type_name(args[0])}")
    else:
        if not _is_dim(args[0]):
            raise TypeError(f"permute() takes 1 positional argument but {len(args)} were given")
        dims = list(args)
    if error is not None:
        raise error
    out = []
    for pos, d in enumerate(dims, 1):
        try:
            v = _operator.index(d)
        except TypeError:
            raise TypeError(f"permute(): argument 'dims' failed to unpack the object at pos {pos} with error "
                            f"\"type must be tuple of ints,but got {_py_type_name(d)}\"") from None
        if not -(2**63) <= v < 2**63:
            raise TypeError(f"permute(): argument 'dims' failed to unpack the object at pos {pos} with error "
                            "\"Overflow when unpacking long long\"")
        out.append(v)
    return out


def _permute(self, *args, **kwargs):
    """Tensor.permute (src/python.rs:823-831, 9512-9553): negative dims are
    normalised here; the view itself is the engine's permute_axes."""
    dims = _permute_dims(args, kwargs)
    rank = len(self.shape)
    if len(dims) != rank:
        raise RuntimeError("permute(sparse_coo): number of dimensions in the tensor input does not match the length "
                           f"of the desired ordering of dimensions i.e. input.dim() = {rank} is not equal to "
                           f"len(dims) = {len(dims)}")
    seen, normalized = set(), []
    for d in dims:
        if d < -rank or d >= rank:
            raise IndexError(f"Dimension out of range (expected to be in range of [{-rank}, {rank - 1}], but got {d})")
        d = d + rank if d < 0 else d
        if d in seen:
            raise RuntimeError("permute(): duplicate dims are not allowed.")
        seen.add(d)
        normalized.append(d)
    return _native_permute(self, *normalized)


Tensor.permute = _permute
Tensor.device = property(_tensor_device)
Tensor.is_cpu = property(lambda self: not self.is_cuda)
Tensor.get_device = lambda self: -1 if not self.is_cuda else int(self._device_str.split(":")[1])
Tensor.to = _to
Tensor.cpu = lambda self: _native_to(self, "cpu")
Tensor.cuda = _cuda
Tensor.tolist = lambda self: self.numpy().tolist()
_native_matmul = Tensor.matmul


def _matmul_method(self, *args, **kwargs):
    """Tensor.matmul(other), also as matmul(other=) or matmul(x2=)."""
    if len(args) == 1 and not kwargs:
        return _native_matmul(self, args[0])
    if not args and len(kwargs) == 1:
        (key, value), = kwargs.items()
        if key in ("other", "x2"):
            return _native_matmul(self, value)
    raise TypeError("matmul() received an invalid combination of arguments")


Tensor.matmul = _matmul_method
Tensor.__array__ = _array
Tensor.__repr__ = _repr
Tensor.__len__ = _len
Tensor.__array_priority__ = 1000.0  # numpy operands defer to the tensor's reflected ops (src/python.rs:3465)
Tensor.__bool__ = _bool
Tensor.multiply = Tensor.mul

from . import accelerator, autograd, compiler, cuda, nn  # noqa: E402,F401
from .fusion import fuse  # noqa: E402,F401
