"""Random operation chains on the device, checked stage by stage against the oracle.

Each chain follows the shape of the reference's chain tests
(tests/test_operation_chains_reference.py:13-159):

    leaf -> input view -> view -> unary -> broadcast mul -> unary -> sum -> backward

The inputs come in four kinds: a scalar, an empty tensor, an offset view
(`leaf[1]`) and a transposed view (`leaf.transpose(0, 2)`).  The views are
transpose, swapdims and squeeze, with dimensions given positive or negative.
The multiplier broadcasts over a random subset of axes.  The unaries are the
hot path's own (neg, exp, relu), chained neg -> exp -> relu -> neg, where the
reference's tests use sin.  The chains are generated here from a seed; they
are not the reference's chains.

What is checked:

- Every stage's values, bit for bit, against the oracle run on the same
  layouts. Exp stages are within 2 ulp of glibc, and everything after them is
  bit-exact, composed from the device's own exp values.
- Every stage's shape, strides (the restated planner), offset and grad_fn
  name.
- The gradients of the leaf and the multiplier, bit for bit.
- The loss within the float summation bound, since the device sums in tree
  order.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
import torch_rs
from helpers import assert_bitwise_equal, ulp_distance

pytestmark = pytest.mark.gpu

SEED = 0x5EED_C4A1
CHAINS = 36
KINDS = ("scalar", "empty", "offset", "transposed")
VIEWS = ("transpose", "swapdims", "squeeze")
UNARIES = ("neg", "exp", "relu")
NEXT = {"neg": "exp", "exp": "relu", "relu": "neg"}
OPCODE = {"neg": O.NEG, "exp": O.EXP, "relu": O.RELU}
NODE = {"neg": "NegBackward0", "exp": "ExpBackward0", "relu": "ReluBackward0"}
LEAF_SHAPE = {"scalar": (), "empty": (2, 0, 3), "offset": (2, 3, 4), "transposed": (2, 3, 4)}


def _chains():
    rng = np.random.default_rng(SEED)
    out = []
    for i in range(CHAINS):
        kind, view, first = KINDS[i % 4], VIEWS[(i // 4) % 3], UNARIES[(i // 12) % 3]
        form = ("operator", "mul", "multiply")[int(rng.integers(0, 3))]
        leaf_shape = LEAF_SHAPE[kind]
        leaf = rng.uniform(-0.75, 0.75, size=leaf_shape).astype(np.float32)
        # Inject a signed zero and exact-zero edge into non-empty leaves.
        if leaf.size >= 2:
            flat = leaf.reshape(-1)
            flat[int(rng.integers(0, flat.size))] = -0.0
            flat[int(rng.integers(0, flat.size))] = 0.0
        in_shape = {"offset": (3, 4), "transposed": (4, 3, 2)}.get(kind, leaf_shape)
        rank = len(in_shape)
        if view == "squeeze":
            dims = None
            v_shape = tuple(d for d in in_shape if d != 1)
        else:
            if rank <= 1:
                a, b = 0, -1
                perm = list(range(rank))
            else:
                a, b = (int(x) for x in rng.choice(rank, size=2, replace=False))
                perm = list(range(rank))
                perm[a], perm[b] = perm[b], perm[a]
                a = a - rank if rng.integers(0, 2) else a
                b = b - rank if rng.integers(0, 2) else b
            dims = (a, b)
            v_shape = tuple(in_shape[p] for p in perm)
        if not v_shape:
            m_shape = (int(rng.integers(2, 5)),)
        else:
            m_shape = [1 if d == 0 else d for d in v_shape]
            for ax, d in enumerate(v_shape):
                if d != 1 and rng.integers(0, 2):
                    m_shape[ax] = 1
            if tuple(m_shape) == v_shape:
                m_shape[next(ax for ax, d in enumerate(v_shape) if d != 1)] = 1
            m_shape = tuple(m_shape)
        mult = (rng.uniform(0.25, 1.25, size=m_shape) * rng.choice([-1.0, 1.0], size=m_shape)).astype(np.float32)
        out.append(dict(kind=kind, view=view, dims=dims, first=first, second=NEXT[first], form=form, leaf=leaf,
                        mult=mult, in_shape=in_shape, v_shape=v_shape))
    return out


def _ids():
    return [f"{c['kind']}-{c['view']}{c['dims'] or ''}-{c['first']}-{c['form']}" for c in _chains()]


def _contig(shape):
    return O.contiguous_strides(shape)


def _storage(logical: np.ndarray, shape, strides) -> np.ndarray:
    """Logical row-major values laid out in a buffer with `strides` (dense)."""
    n = O.storage_size(shape, strides)
    buf = np.zeros(max(n, 1), np.float32)
    if logical.size:
        view = np.lib.stride_tricks.as_strided(buf, shape=shape, strides=tuple(4 * s for s in strides))
        view[...] = logical.reshape(shape)
    return buf


def _logical(buf, shape, strides, off=0) -> np.ndarray:
    if not shape:
        return buf[off:off + 1].copy()
    n = int(np.prod(shape))
    if n == 0:
        return np.zeros(0, np.float32)
    return O.unary(O.COPY, buf, shape, strides, off, _contig(shape))[:n]


def _layout_of(t):
    return tuple(t.shape), tuple(t.stride()), t.storage_offset()


def _input_layout(c):
    if c["kind"] == "offset":
        return (3, 4), (4, 1), 12
    if c["kind"] == "transposed":
        return (4, 3, 2), (1, 4, 12), 0
    return c["leaf"].shape, _contig(c["leaf"].shape), 0


def _view_layout(c, shape, strides, off):
    if c["view"] == "squeeze":
        keep = [i for i, d in enumerate(shape) if d != 1]
        return tuple(shape[i] for i in keep), tuple(strides[i] for i in keep), off, None
    rank = len(shape)
    perm = list(range(rank))
    if rank >= 2:
        a, b = (d % rank for d in c["dims"])
        perm[a], perm[b] = perm[b], perm[a]
    return tuple(shape[p] for p in perm), tuple(strides[p] for p in perm), off, perm


def _unary_vjp(name, up, inp_buf, shape, strides, off, out_logical):
    if name == "neg":
        return O.unary_contig(O.NEG, up)
    if name == "relu":
        return O.relu_backward(inp_buf, shape, strides, off, up)
    return O.binary_contig(O.MUL, up, out_logical)  # exp: up * exp(x), one rounding


@pytest.mark.parametrize("c", _chains(), ids=_ids())
def test_chain_matches_oracle_stage_by_stage(c):
    # ---- device forward ------------------------------------------------------
    leaf = torch_rs.tensor(c["leaf"], device="cuda", requires_grad=True)
    inp = leaf[1] if c["kind"] == "offset" else leaf.transpose(0, 2) if c["kind"] == "transposed" else leaf
    view = inp.squeeze() if c["view"] == "squeeze" else getattr(inp, c["view"])(*c["dims"])
    u1 = getattr(view, c["first"])()
    mult = torch_rs.tensor(c["mult"], device="cuda", requires_grad=True)
    m = u1 * mult if c["form"] == "operator" else getattr(u1, c["form"])(mult)
    u2 = getattr(m, c["second"])()
    loss = u2.sum()
    loss.backward()

    # ---- oracle, stage by stage ---------------------------------------------
    leaf_buf = c["leaf"].reshape(-1) if c["leaf"].size else np.zeros(1, np.float32)
    i_shape, i_str, i_off = _input_layout(c)
    assert _layout_of(inp) == (tuple(i_shape), tuple(i_str), i_off)
    v_shape, v_str, v_off, perm = _view_layout(c, i_shape, i_str, i_off)
    assert _layout_of(view) == (v_shape, v_str, v_off)
    assert view.grad_fn.name() == ("SqueezeBackward0" if c["view"] == "squeeze" else "TransposeBackward0")

    def check_unary(name, dev, src_buf, shape, strides, off):
        o_str = O.unary_output_strides(shape, strides)
        want = O.unary(OPCODE[name], src_buf, shape, strides, off, o_str)
        assert _layout_of(dev) == (tuple(shape), o_str, 0)
        assert dev.grad_fn.name() == NODE[name]
        got = dev.numpy().reshape(-1)
        want_logical = _logical(want, shape, o_str)
        if name == "exp":
            if got.size:
                assert ulp_distance(got, want_logical).max() <= 2
            return _storage(got, shape, o_str), o_str, got  # downstream uses the device's exp values
        assert_bitwise_equal(got, want_logical)
        return want, o_str, want_logical

    u1_buf, u1_str, u1_log = check_unary(c["first"], u1, leaf_buf, v_shape, v_str, v_off)

    mt_shape = c["mult"].shape
    m_shape, m_str = O.binary_output_layout(v_shape, u1_str, mt_shape, _contig(mt_shape))
    m_buf = O.binary(O.MUL, u1_buf, v_shape, u1_str, 0, c["mult"].reshape(-1), mt_shape, _contig(mt_shape), 0,
                     m_shape, m_str)
    assert _layout_of(m) == (tuple(m_shape), tuple(m_str), 0)
    assert m.grad_fn.name() == "MulBackward0"
    assert_bitwise_equal(m.numpy().reshape(-1), _logical(m_buf, m_shape, m_str))

    u2_buf, u2_str, u2_log = check_unary(c["second"], u2, m_buf, m_shape, m_str, 0)

    n2 = int(np.prod(m_shape))
    want_loss = O.sum_f32(u2_buf, m_shape, u2_str, 0)
    bound = n2 * 2.0 ** -24 * float(np.abs(u2_log).sum())
    assert abs(float(loss.item()) - float(want_loss)) <= bound
    assert loss.grad_fn.name() == "SumBackward0"

    # ---- backward: each VJP in the reference's order ----------------------------
    up2 = np.ones(n2, np.float32)
    d_m = _unary_vjp(c["second"], up2, m_buf, m_shape, m_str, 0, u2_log)
    d_u1 = O.mul_backward(d_m, m_shape, c["mult"].reshape(-1), mt_shape, _contig(mt_shape), 0, v_shape)
    d_mult = O.mul_backward(d_m, m_shape, u1_buf, v_shape, u1_str, 0, mt_shape)
    d_view = _unary_vjp(c["first"], d_u1, leaf_buf, v_shape, v_str, v_off, u1_log)
    if perm is None:
        d_inp = d_view
    else:
        d_inp = O.permute_backward(d_view, v_shape, perm, i_shape)
    if c["kind"] == "offset":
        d_leaf = np.zeros(c["leaf"].shape, np.float32)
        d_leaf[1] = d_inp.reshape(i_shape)
    elif c["kind"] == "transposed":
        d_leaf = O.permute_backward(d_inp, i_shape, (2, 1, 0), c["leaf"].shape)
    else:
        d_leaf = d_inp

    assert leaf.grad.shape == c["leaf"].shape
    assert mult.grad.shape == mt_shape
    n_leaf = c["leaf"].size
    assert_bitwise_equal(leaf.grad.numpy().reshape(-1), np.asarray(d_leaf, np.float32).reshape(-1)[:n_leaf])
    assert_bitwise_equal(mult.grad.numpy().reshape(-1), d_mult[: c["mult"].size])


def test_scalar_subtraction_records_the_reference_node_name():
    x = torch_rs.tensor(np.float32([1.5, -2.0]), device="cuda", requires_grad=True)
    assert (x - 1.0).grad_fn.name() == "SubBackward0"
    assert (1.0 - x).grad_fn.name() == "RsubBackward1"


def test_squeeze_dims_gradient_maps_back_to_the_input_shape():
    x = torch_rs.tensor(np.arange(6, dtype=np.float32).reshape(1, 2, 1, 3), device="cuda", requires_grad=True)
    y = x.squeeze((0, 2))
    assert y.shape == (2, 3) and y.grad_fn.name() == "SqueezeBackward2"
    w = torch_rs.tensor(np.float32([[1, 2, 3], [4, 5, 6]]), device="cuda")
    (y * w).sum().backward()
    assert x.grad.shape == (1, 2, 1, 3)
    assert x.grad.numpy().reshape(-1).tolist() == [1, 2, 3, 4, 5, 6]
    z = torch_rs.tensor(np.ones((2, 1), np.float32), device="cuda", requires_grad=True)
    s = z.squeeze(-1)
    assert s.shape == (2,) and s.grad_fn.name() == "SqueezeBackward1"
    s.sum().backward()
    assert z.grad.numpy().tolist() == [[1.0], [1.0]]
