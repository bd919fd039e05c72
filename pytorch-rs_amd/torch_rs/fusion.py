"""torch_rs.fuse -- the pointwise fusion front end.

``fuse(fn)`` traces ``fn`` (a function of tensors built from + - * /, scalar
operands, exp, relu and neg; a device byte buffer such as a dropout keep-mask
may stand in for a tensor and is read as 0/1 floats) into the pointwise IR of
libtrs_hip.so's
fusion compiler, which emits HIP C++ and compiles it with hipRTC for gfx950
into ONE kernel.  Every IR instruction rounds exactly as the eager op it
stands for, so the fused result is the eager chain's result (bit for bit
where the chain has no exp).  The output layout is the one the eager chain
would produce: the tracer runs the same output-stride planner
(elementwise_output_strides and friends, src/tensor.rs:4249-4312) op by op.

The reference has no fusion (torch.jit.strict_fusion is a warning-only
no-op, README.md:178); this component is new.

Calls whose inputs need gradients record the fused launch as one graph node
(FusedBackward0).  Its backward is generated from the same IR by reverse
mode: ONE fused program with an output per input that needs a gradient,
recomputing the forward values and applying, per element, exactly the
roundings of the eager VJPs (up * other for mul, up * exp(x) for exp, relu'
for relu, sign flips for neg and reflected sub; division records nothing, as
in the reference).  Broadcast inputs are then reduced in the reference's
order.  That reproduces eager autograd bit for bit when every value the
gradient reaches has the output's shape, no such value feeds more than two
gradient-carrying uses (two contributions add commutatively) and each
broadcast input feeds at most one; other programs run ``fn`` eagerly so
autograd records op by op.
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
    """Instructions in definition order: ("in", i), ("const", bits), (op, a[, b]);
    `shapes` holds the eager shape of every traced (non-constant) value."""

    def __init__(self, u8=()):
        self.ins: list[tuple] = []
        self.consts: dict[str, int] = {}
        self.shapes: dict[int, tuple] = {}
        self.u8 = set(u8)  # input positions read as bytes ("in u8")

    def emit(self, *instr) -> int:
        self.ins.append(instr)
        return len(self.ins) - 1

    def const(self, v) -> int:
        return self.const_bits(_f32_bits(v))

    def const_bits(self, bits: str) -> int:
        if bits not in self.consts:
            self.consts[bits] = self.emit("const", bits)
        return self.consts[bits]

    def live(self, outs) -> set:
        """The values the output(s) `outs` depend on."""
        live = set()
        stack = [outs] if isinstance(outs, int) else list(outs)
        while stack:
            v = stack.pop()
            if v in live:
                continue
            live.add(v)
            ins = self.ins[v]
            if ins[0] not in ("in", "const"):
                stack.extend(ins[1:])
        return live

    def _numel(self, v) -> int:
        n = 1
        for d in self.shapes.get(v, ()):
            n *= d
        return n

    def finish(self, outs):
        """IR text of the instructions the output(s) `outs` depend on,
        renumbered, and the argument positions of the inputs it reads (dead
        code and unused inputs are dropped, so they are neither loaded nor
        required to broadcast to the output shape).

        Inputs smaller than the output (broadcast, re-read from cache) are
        declared before the full-size ones: a kernel issues its loads in
        input order, and issuing the cached loads before the streaming ones
        measured 2-3% faster on a row-broadcast add.  The instructions still
        take their operands in traced order, so the arithmetic is unchanged."""
        outs = [outs] if isinstance(outs, int) else list(outs)
        live = self.live(outs)
        full = max(self._numel(o) for o in outs)
        inputs = [v for v, ins in enumerate(self.ins) if v in live and ins[0] == "in"]
        if all(v in self.shapes for v in inputs):
            inputs.sort(key=lambda v: self._numel(v) >= full)  # stable: broadcast first
        new_id, lines, used_inputs = {}, [], []
        for v in inputs:
            new_id[v] = len(lines)
            used_inputs.append(self.ins[v][1])
            lines.append("in u8" if self.ins[v][1] in self.u8 else "in f32")
        for v, ins in enumerate(self.ins):
            if v not in live or ins[0] == "in":
                continue
            new_id[v] = len(lines)
            if ins[0] == "const":
                lines.append(f"const {ins[1]}")
            else:
                lines.append(ins[0] + "".join(f" %{new_id[a]}" for a in ins[1:]))
        lines.extend(f"out %{new_id[o]}" for o in outs)
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
        tr.shapes[vid] = self.shape

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


_NO_GRAD = "no-grad"


def _gradient_program(tr, out, requires, out_shape):
    """The backward IR of a traced program, or None when the program needs the
    eager path for bit-exact gradients, or _NO_GRAD when the output records
    nothing (every path to it goes through a division).

    `requires[i]`: input i requires grad.  Returns (IR text, argument list,
    targets): an argument is an input position or -1 for the upstream
    gradient; output o of the program is the gradient of input targets[o]."""
    ins = tr.ins
    live = sorted(tr.live(out))
    rg = {}
    for v in live:
        op = ins[v][0]
        if op == "in":
            rg[v] = bool(requires[ins[v][1]])
        elif op in ("const", "div"):
            rg[v] = False
        elif op in ("add", "sub", "mul"):
            rg[v] = rg[ins[v][1]] or rg[ins[v][2]]
        else:  # exp, relu, neg
            rg[v] = rg[ins[v][1]]
    if not rg[out]:
        return _NO_GRAD
    # The values a gradient reaches from the output (never through a
    # division, which records nothing), and their gradient-carrying uses.
    reach = {out}
    uses: dict[int, int] = {}
    for u in reversed(live):
        if u not in reach or ins[u][0] in ("in", "const"):
            continue
        for a in ins[u][1:]:
            if rg[a]:
                reach.add(a)
                uses[a] = uses.get(a, 0) + 1
    for v in reach:
        full = tr.shapes.get(v) == tuple(out_shape)
        if ins[v][0] == "in":
            # A broadcast input reduces each contribution on its own in eager
            # autograd, so it may have only one; a full-shape input may have
            # two, which add commutatively as the engine accumulates them.
            if uses.get(v, 0) > (2 if full else 1):
                return None
        elif not full or uses.get(v, 0) > 2:
            return None

    n_in = len(requires)  # the upstream gradient's argument slot
    bt = _Trace(tr.u8)
    fwd = {}
    for u in live:  # the forward values, recomputed
        i = ins[u]
        if i[0] == "in":
            fwd[u] = bt.emit("in", i[1])
        elif i[0] == "const":
            fwd[u] = bt.const_bits(i[1])
        else:
            fwd[u] = bt.emit(i[0], *(fwd[a] for a in i[1:]))
    adj = {out: bt.emit("in", n_in)}  # the upstream gradient

    def contribute(x, val):
        if not rg[x]:
            return
        adj[x] = bt.emit("add", adj[x], val) if x in adj else val

    for u in reversed(live):
        if u not in adj or ins[u][0] in ("in", "const"):
            continue
        g, (op, *args) = adj[u], ins[u]
        if op == "add":
            contribute(args[0], g)
            contribute(args[1], g)
        elif op == "sub":
            contribute(args[0], g)
            if rg[args[1]]:
                contribute(args[1], bt.emit("neg", g))
        elif op == "mul":
            if rg[args[0]]:
                contribute(args[0], bt.emit("mul", g, fwd[args[1]]))
            if rg[args[1]]:
                contribute(args[1], bt.emit("mul", g, fwd[args[0]]))
        elif op == "exp":
            contribute(args[0], bt.emit("mul", g, fwd[u]))
        elif op == "relu":
            contribute(args[0], bt.emit("relub", fwd[args[0]], g))
        elif op == "neg":
            contribute(args[0], bt.emit("neg", g))
    inputs = [v for v in live if ins[v][0] == "in" and v in reach]
    ir, used = bt.finish([adj[v] for v in inputs])
    return ir, [-1 if i == n_in else i for i in used], [ins[v][1] for v in inputs]


class Fused:
    """A traced-and-compiled pointwise function (see the module docstring)."""

    def __init__(self, fn):
        self.fn = fn
        self._cache: dict = {}
        functools.update_wrapper(self, fn)

    def _trace(self, inputs):
        tr = _Trace(i for i, t in enumerate(inputs) if isinstance(t, _C.ByteBuffer))
        proxies = []
        for i, t in enumerate(inputs):
            proxies.append(_Proxy(tr, tr.emit("in", i), t.shape, _strides(t)))
        out = self.fn(*proxies)
        if not isinstance(out, _Proxy):
            raise TypeError("a fused function must return a traced tensor expression")
        if tr.ins[out.vid][0] == "in":
            raise TypeError("a fused function must compute something from its inputs")
        return tr, out

    def trace(self, *inputs):
        """(IR text, output shape, output strides, positions of the inputs the
        output reads) for inputs of these layouts."""
        tr, out = self._trace(inputs)
        ir, used = tr.finish(out.vid)
        return ir, out.shape, out.strides, used

    def program(self, *inputs):
        key = _layout_key(inputs)
        hit = self._cache.get(key)
        if hit is None:
            ir, shape, strides, used = self.trace(*inputs)
            hit = (_C.FusedProgram.compile(ir, len(used)), list(shape), list(strides), used, ir)
            self._cache[key] = hit
        return hit

    def grad_plan(self, *inputs):
        """None (eager autograd), _NO_GRAD, or the gradient program as
        (compiled program id, argument positions among the forward's inputs
        or -1 for the upstream, the forward input position of each output)."""
        requires = tuple(bool(getattr(t, "requires_grad", False)) for t in inputs)
        key = (_layout_key(inputs), requires)
        if key in self._cache:
            return self._cache[key]
        tr, out = self._trace(inputs)
        plan = _gradient_program(tr, out.vid, requires, out.shape)
        if isinstance(plan, tuple):
            ir, args, targets = plan
            _, _, _, used, _ = self.program(*inputs)
            pos = {orig: p for p, orig in enumerate(used)}
            plan = (_C.FusedProgram.compile(ir, len(args)).id, [-1 if a < 0 else pos[a] for a in args],
                    [pos[t] for t in targets])
        self._cache[key] = plan
        return plan

    def __call__(self, *inputs):
        if not inputs or not all(isinstance(t, (_C.Tensor, _C.ByteBuffer)) for t in inputs):
            raise TypeError("fused functions take tensors (or device byte buffers) only; bind scalars in the "
                            "function body")
        prog, shape, strides, used, _ = self.program(*inputs)
        args = [inputs[i] for i in used]
        if _C.is_grad_enabled() and any(getattr(t, "requires_grad", False) for t in inputs):
            plan = self.grad_plan(*inputs)
            if plan is None:
                return self.fn(*inputs)
            if plan != _NO_GRAD:
                return prog.launch_with_grad(args, shape, strides, *plan)
        return prog.launch(args, shape, strides)


def _strides(t) -> tuple:
    if isinstance(t, _C.ByteBuffer):
        return tuple(_L.contiguous_strides(list(t.shape)))
    return t.stride()


def _layout_key(inputs) -> tuple:
    return tuple(("u8" if isinstance(t, _C.ByteBuffer) else "f32", tuple(t.shape), tuple(_strides(t)))
                 for t in inputs)


def fuse(fn):
    """Decorator: compile ``fn`` into one pointwise kernel per input layout."""
    return Fused(fn)
