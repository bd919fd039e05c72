"""torch_rs.fuse -- the pointwise fusion front end.

``fuse(fn)`` traces ``fn`` (a function of tensors built from + - * /, scalar
operands, exp, relu and neg) into the pointwise IR of libtrs_hip.so's
fusion compiler, which emits HIP C++ and compiles it with hipRTC for gfx950
into ONE kernel.  Every IR instruction rounds exactly as the eager op it
stands for, so the fused result is the eager chain's result (bit for bit
where the chain has no exp).  The output layout is the one the eager chain
would produce: the tracer runs the same output-stride planner
(elementwise_output_strides and friends, src/tensor.rs:4249-4312) op by op.

The reference has no fusion (torch.jit.strict_fusion is a warning-only
no-op, README.md:178); this component is new.  Calls whose inputs need
gradients run ``fn`` eagerly instead, so autograd records as usual.
"""
from __future__ import annotations

import functools
import struct

import numpy as _np

from ._native import native as _C

_L = _C.layout


def _f32_bits(v) -> str:
    return "0x%08x" % struct.unpack("<I", struct.pack("<f", _np.float32(v)))[0]


class _Trace:
    """Instructions in definition order: ("in", i), ("const", bits), (op, a[, b])."""

    def __init__(self):
        self.ins: list[tuple] = []
        self.consts: dict[str, int] = {}

    def emit(self, *instr) -> int:
        self.ins.append(instr)
        return len(self.ins) - 1

    def const(self, v) -> int:
        bits = _f32_bits(v)
        if bits not in self.consts:
            self.consts[bits] = self.emit("const", bits)
        return self.consts[bits]

    def finish(self, out: int):
        """IR text of the instructions `out` depends on, renumbered, and the
        argument positions of the inputs it reads (dead code and unused
        inputs are dropped, so they are neither loaded nor required to
        broadcast to the output shape)."""
        live = set()
        stack = [out]
        while stack:
            v = stack.pop()
            if v in live:
                continue
            live.add(v)
            ins = self.ins[v]
            if ins[0] not in ("in", "const"):
                stack.extend(ins[1:])
        new_id, lines, used_inputs = {}, [], []
        for v, ins in enumerate(self.ins):
            if v not in live:
                continue
            new_id[v] = len(lines)
            if ins[0] == "in":
                used_inputs.append(ins[1])
                lines.append("in f32")
            elif ins[0] == "const":
                lines.append(f"const {ins[1]}")
            else:
                lines.append(ins[0] + "".join(f" %{new_id[a]}" for a in ins[1:]))
        lines.append(f"out %{new_id[out]}")
        return "\n".join(lines) + "\n", used_inputs


def _scalar(v):
    if isinstance(v, bool):
        return _np.float32(1.0 if v else 0.0)
    if isinstance(v, (int, float, _np.integer, _np.floating)):
        return _np.float32(v)
    return None


class _Proxy:
    """A traced value: IR id plus the (shape, strides) the eager op would produce."""

    __slots__ = ("tr", "vid", "shape", "strides")

    def __init__(self, tr, vid, shape, strides):
        self.tr, self.vid, self.shape, self.strides = tr, vid, tuple(shape), tuple(strides)

    def _numel(self):
        n = 1
        for d in self.shape:
            n *= d
        return n

    def _binary(self, other, op, reverse=False):
        if isinstance(other, _Proxy):
            l, r = (other, self) if reverse else (self, other)
            shape, strides = _L.binary_output_layout(list(l.shape), list(l.strides), list(r.shape), list(r.strides))
            return _Proxy(self.tr, self.tr.emit(op, l.vid, r.vid), shape, strides)
        s = _scalar(other)
        if s is None:
            return NotImplemented
        if op == "sub" and isinstance(other, bool):
            raise RuntimeError("Subtraction, the `-` operator, with a bool tensor is not supported. If you are "
                               "trying to invert a mask, use the `~` or `logical_not()` operator instead.")
        c = self.tr.const(s)
        strides = _L.scalar_output_strides(list(self.shape), list(self.strides))
        if op == "div" and reverse:  # scalar_div: s * (1 / v) (src/tensor.rs:2316-2339)
            ustr = _L.unary_output_strides(list(self.shape), list(self.strides), self._numel())
            strides = _L.elementwise_output_strides(list(self.shape), [(list(self.shape), list(ustr))])
            one = self.tr.const(1.0)
            rec = self.tr.emit("div", one, self.vid)
            return _Proxy(self.tr, self.tr.emit("mul", c, rec), self.shape, strides)
        a, b = (c, self.vid) if reverse else (self.vid, c)
        if op in ("add", "mul") and reverse:
            a, b = self.vid, c  # v + s and v * s, as add_scalar / mul_scalar compute them
        return _Proxy(self.tr, self.tr.emit(op, a, b), self.shape, strides)

    def _unary(self, op):
        strides = _L.unary_output_strides(list(self.shape), list(self.strides), self._numel())
        return _Proxy(self.tr, self.tr.emit(op, self.vid), self.shape, strides)

    __add__ = lambda self, o: self._binary(o, "add")
    __radd__ = lambda self, o: self._binary(o, "add", True)
    __sub__ = lambda self, o: self._binary(o, "sub")
    __rsub__ = lambda self, o: self._binary(o, "sub", True)
    __mul__ = lambda self, o: self._binary(o, "mul")
    __rmul__ = lambda self, o: self._binary(o, "mul", True)
    __truediv__ = lambda self, o: self._binary(o, "div")
    __rtruediv__ = lambda self, o: self._binary(o, "div", True)
    __neg__ = lambda self: self._unary("neg")
    add = __add__
    sub = __sub__
    mul = __mul__
    div = __truediv__
    neg = __neg__

    def exp(self):
        return self._unary("exp")

    def relu(self):
        return self._unary("relu")


class Fused:
    """A traced-and-compiled pointwise function (see the module docstring)."""

    def __init__(self, fn):
        self.fn = fn
        self._cache: dict = {}
        functools.update_wrapper(self, fn)

    def trace(self, *inputs):
        """(IR text, output shape, output strides, positions of the inputs the
        output reads) for inputs of these layouts."""
        tr = _Trace()
        proxies = []
        for i, t in enumerate(inputs):
            proxies.append(_Proxy(tr, tr.emit("in", i), t.shape, t.stride()))
        out = self.fn(*proxies)
        if not isinstance(out, _Proxy):
            raise TypeError("a fused function must return a traced tensor expression")
        if tr.ins[out.vid][0] == "in":
            raise TypeError("a fused function must compute something from its inputs")
        ir, used = tr.finish(out.vid)
        return ir, out.shape, out.strides, used

    def program(self, *inputs):
        key = tuple((t.shape, t.stride()) for t in inputs)
        hit = self._cache.get(key)
        if hit is None:
            ir, shape, strides, used = self.trace(*inputs)
            hit = (_C.FusedProgram.compile(ir, len(used)), list(shape), list(strides), used, ir)
            self._cache[key] = hit
        return hit

    def __call__(self, *inputs):
        if not inputs or not all(isinstance(t, _C.Tensor) for t in inputs):
            raise TypeError("fused functions take tensors only (bind scalars in the function body)")
        if _C.is_grad_enabled() and any(t.requires_grad for t in inputs):
            return self.fn(*inputs)
        prog, shape, strides, used, _ = self.program(*inputs)
        return prog.launch([inputs[i] for i in used], shape, strides)


def fuse(fn):
    """Decorator: compile ``fn`` into one pointwise kernel per input layout."""
    return Fused(fn)
