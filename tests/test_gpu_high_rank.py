"""Views above the kernels' eight dims, through the C ABI and torch_rs.

The reference's shapes are vectors of any length (src/tensor.rs:212-221).
The ABI takes up to TRS_MAX_RANK (25) dims; a kernel's geometry indexes at
most 8 after size-1 dims are dropped and contiguous dims merged.  A
pointwise view that keeps more is run as one launch per index tuple of its
outermost dims, sum copies such a view to a contiguous buffer first, and the
broadcast reduction merges its kept and reduced dims, walking any number that
remain.

The views here are built so that nothing merges: an operand transposed in
every dim (a contiguous buffer of the reversed shape, read in reverse dim
order) next to a contiguous one.  Bar: bit-exact against the oracle on the
same layouts, exp within 2 ulp of glibc, as at lower rank.
"""
import ctypes
import zlib

import numpy as np
import pytest

import gpu_util as U
import oracle as O
import torch_rs
from helpers import assert_bitwise_equal, ulp_distance
from trs_backend import abi
from trs_backend.abi import check, layout_of

pytestmark = pytest.mark.gpu

SHAPES = {
    8: (2, 3, 2, 3, 2, 3, 2, 5),  # no split: all 8 dims in the kernel's geometry
    9: (2, 3, 2, 3, 2, 3, 2, 3, 2),
    10: (3, 2, 3, 2, 3, 2, 3, 2, 3, 5),
    12: (2, 3) * 6,
    16: (2,) * 15 + (7,),
    25: (2,) * 12 + (1,) * 10 + (3, 1, 2),
}


def reversed_strides(shape):
    """Strides of a view transposed in every dim: dim d of the view is dim
    rank-1-d of a contiguous buffer of the reversed shape."""
    return tuple(reversed(O.contiguous_strides(tuple(reversed(shape)))))


def rng_for(name):
    return np.random.default_rng(zlib.crc32(name.encode()))


def plan_split(layouts, out):
    return abi.pointwise_plan(list(layouts), out).split


@pytest.mark.parametrize("rank", sorted(SHAPES))
@pytest.mark.parametrize("op", [O.ADD, O.MUL, O.DIV])
def test_binary_with_a_reversed_operand(rank, op):
    shape = SHAPES[rank]
    n = int(np.prod(shape))
    rng = rng_for(f"bin{rank}{op}")
    a, b = U.special_mix(rng, n), U.special_mix(rng, n)
    ast, bst = O.contiguous_strides(shape), reversed_strides(shape)
    oshape, ostr = O.binary_output_layout(shape, ast, shape, bst)
    nonunit = sum(1 for d in shape if d != 1)
    assert plan_split([layout_of(shape, ast), layout_of(shape, bst)], layout_of(oshape, ostr)) == max(0, nonunit - 8)
    want = O.binary(op, a, shape, ast, 0, b, shape, bst, 0, oshape, ostr)
    got = U.binary(op, a, shape, ast, 0, b, shape, bst, 0, oshape, ostr)
    assert_bitwise_equal(got, want)


@pytest.mark.parametrize("rank", [10, 12])
def test_broadcast_operand_and_offset_output_order_of_the_first_operand(rank):
    """The reversed operand comes first, so the output takes its dim order
    (the reference's output-stride rule); the other operand broadcasts along
    every third dim and starts at an offset."""
    shape = SHAPES[rank]
    rng = rng_for(f"bc{rank}")
    bshape = tuple(1 if d % 3 == 1 else s for d, s in enumerate(shape))
    n, nb = int(np.prod(shape)), int(np.prod(bshape))
    a = U.special_mix(rng, n)
    b = U.special_mix(rng, nb + 3)
    ast, bst = reversed_strides(shape), O.contiguous_strides(bshape)
    oshape, ostr = O.binary_output_layout(shape, ast, bshape, bst)
    assert ostr == ast
    for op in (O.ADD, O.SUB, O.MUL):
        want = O.binary(op, a, shape, ast, 0, b, bshape, bst, 3, oshape, ostr)
        got = U.binary(op, a, shape, ast, 0, b, bshape, bst, 3, oshape, ostr)
        assert_bitwise_equal(got, want)


@pytest.mark.parametrize("rank", [8, 9, 12, 25])
def test_unary_and_scalar_ops_on_a_reversed_view(rank):
    shape = SHAPES[rank]
    n = int(np.prod(shape))
    rng = rng_for(f"un{rank}")
    a = U.special_mix(rng, n)
    st = reversed_strides(shape)
    ostr = O.contiguous_strides(shape)
    for op in (O.COPY, O.NEG, O.RELU):
        assert_bitwise_equal(U.unary(op, a, shape, st, 0, ostr), O.unary(op, a, shape, st, 0, ostr))
    got = U.unary(O.EXP, a, shape, st, 0, ostr)
    want = O.unary(O.EXP, a, shape, st, 0, ostr)
    fin = np.isfinite(want)
    assert (np.isnan(got) == np.isnan(want)).all()
    assert ulp_distance(got[fin], want[fin]).max() <= 2
    s = float(np.float32(1.0 / 0.9))
    for op in (O.S_MUL, O.S_RSUB):
        assert_bitwise_equal(U.scalar(op, a, shape, st, 0, s, ostr), O.scalar(op, a, shape, st, 0, s, ostr))


def test_mask_apply_on_views_above_eight_dims():
    shape = SHAPES[10]
    n = int(np.prod(shape))
    rng = rng_for("mask")
    h = U.special_mix(rng, n)
    mask = (rng.random(n) < 0.9).astype(np.uint8)
    hst = reversed_strides(shape)
    s = float(np.float32(1.0 / 0.9))
    dh, dm = U.dev(h), U.dev(mask)
    out = U.out_buffer(n)
    check(abi.lib.trs_mask_apply_f32(dh.ptr, ctypes.byref(layout_of(shape, hst)), dm.ptr,
                                     ctypes.byref(layout_of(shape)), ctypes.c_float(s), out.ptr,
                                     ctypes.byref(layout_of(shape))))
    logical_h = O.unary(O.COPY, h, shape, hst, 0, O.contiguous_strides(shape))
    assert_bitwise_equal(out.to_numpy(count=n), O.mask_apply(logical_h, mask, s))


def test_fused_program_above_eight_dims():
    """(a + b) * c with b broadcast and c reversed, in one fused launch per
    part, equals the eager oracle composition bit for bit."""
    shape = SHAPES[12]
    rng = rng_for("fused")
    bshape = tuple(1 if d % 2 == 0 else s for d, s in enumerate(shape))
    n, nb = int(np.prod(shape)), int(np.prod(bshape))
    a, b, c = U.special_mix(rng, n), U.special_mix(rng, nb), U.special_mix(rng, n)
    ast, bst, cst = O.contiguous_strides(shape), O.contiguous_strides(bshape), reversed_strides(shape)
    lays = [layout_of(shape, ast), layout_of(bshape, bst), layout_of(shape, cst)]
    assert plan_split(lays, layout_of(shape)) == 4
    kid = U.fusion_compile("in f32\nin f32\nin f32\nadd %0 %1\nmul %3 %2\nout %4\n")
    out = U.out_buffer(n)
    U.fusion_launch(kid, [U.dev(a), U.dev(b), U.dev(c)], lays, out, layout_of(shape))
    t = O.binary(O.ADD, a, shape, ast, 0, b, bshape, bst, 0, shape, ast)
    want = O.binary(O.MUL, t, shape, ast, 0, c, shape, cst, 0, shape, ast)
    assert_bitwise_equal(out.to_numpy(count=n), want)


def _sum(buf, shape, strides, noalloc=False):
    out = U.out_buffer(1)
    fn = abi.lib.trs_sum_f32_noalloc if noalloc else abi.lib.trs_sum_f32
    rc = fn(buf.ptr, ctypes.byref(layout_of(shape, strides)), out.ptr)
    return rc, out.to_numpy(count=1)[0]


@pytest.mark.parametrize("rank", [8, 10, 16])
def test_sum_of_a_view_that_keeps_more_than_eight_dims(rank):
    """The device sums by logical position, so a view's sum equals, bit for
    bit, the sum of the same values laid out contiguously.  A view keeping 8
    dims is decoded in place; above 8 it is copied first, which the
    no-allocation entry point cannot do, so that one refuses it."""
    shape = SHAPES[rank]
    n = int(np.prod(shape))
    rng = rng_for(f"sum{rank}")
    a = rng.standard_normal(n).astype(np.float32)
    st = reversed_strides(shape)
    logical = O.unary(O.COPY, a, shape, st, 0, O.contiguous_strides(shape))
    rc, got = _sum(U.dev(a), shape, st)
    check(rc)
    rc2, want = _sum(U.dev(logical), (n,), (1,))
    check(rc2)
    assert_bitwise_equal(np.float32([got]), np.float32([want]))
    # the tree's documented depth bound (include/trs_hip.h, trs_sum_f32)
    depth = -(-n // 256) + 8 if n <= 32768 else -(-(-(-n // 1024)) // 256) + 20
    u = 2.0 ** -24
    exact = float(np.sum(logical.astype(np.float64)))
    bound = depth * u / (1 - depth * u) * float(np.sum(np.abs(logical.astype(np.float64))))
    assert abs(float(got) - exact) <= bound
    rc3, got3 = _sum(U.dev(a), shape, st, noalloc=True)
    if rank > 8:
        assert rc3 == abi.TRS_E_INVALID_ARGUMENT
    else:
        check(rc3)
        assert_bitwise_equal(np.float32([got3]), np.float32([want]))
    # a contiguous view of the same rank merges to one dim: no copy needed
    rc4, got4 = _sum(U.dev(logical), shape, O.contiguous_strides(shape), noalloc=True)
    check(rc4)
    assert_bitwise_equal(np.float32([got4]), np.float32([want]))


def gpu_mul_backward(up, oshape, other, oth_shape, oth_strides, self_shape):
    n = int(np.prod(self_shape))
    du, dother = U.dev(up), U.dev(other)
    out = U.out_buffer(n)
    rc = abi.lib.trs_mul_backward_f32(du.ptr, ctypes.byref(layout_of(oshape)), dother.ptr,
                                      ctypes.byref(layout_of(oth_shape, oth_strides)),
                                      ctypes.byref(layout_of(self_shape)), out.ptr)
    return rc, out.to_numpy(count=n)


@pytest.mark.parametrize("rank", [10, 12])
def test_broadcast_reduction_above_eight_dims(rank):
    """The multiply VJP for an operand broadcast along every third dim of a
    rank-10/12 output, the other operand reversed: kept and reduced dims
    merge to at most 8 each, and the accumulation order is the reference's."""
    shape = SHAPES[rank]
    rng = rng_for(f"red{rank}")
    self_shape = tuple(1 if d % 3 == 1 else s for d, s in enumerate(shape))
    n = int(np.prod(shape))
    up = rng.standard_normal(n).astype(np.float32)
    other = U.special_mix(rng, n)
    ost = reversed_strides(shape)
    rc, got = gpu_mul_backward(up, shape, other, shape, ost, self_shape)
    check(rc)
    want = O.mul_backward(up, shape, other, shape, ost, 0, self_shape)
    assert_bitwise_equal(got, want)


def test_broadcast_reduction_whose_dims_do_not_merge():
    """Kept and reduced dims alternating 9 times each (rank 18), and a
    reversed other operand at rank 12 that merges nothing: the per-element
    reduction walks any number of dims in the reference's order."""
    rng = rng_for("alternating")
    for shape, self_shape, ost in [((2, 2) * 9, (2, 1) * 9, None),
                                   ((2, 3) * 6, (1, 3) + (2, 3) * 5, reversed_strides((2, 3) * 6))]:
        n = int(np.prod(shape))
        ost = ost or O.contiguous_strides(shape)
        up = rng.standard_normal(n).astype(np.float32)
        other = U.special_mix(rng, n)
        rc, got = gpu_mul_backward(up, shape, other, shape, ost, self_shape)
        check(rc)
        assert_bitwise_equal(got, O.mul_backward(up, shape, other, shape, ost, 0, self_shape))


def test_torch_rs_autograd_on_rank_ten_tensors():
    """relu(x * w.permute(reversed)).sum() on rank-10 device tensors: the
    forward values and both gradients bit for bit against float32 numpy,
    whose elementwise products are IEEE single roundings like the
    reference's."""
    shape = SHAPES[10]
    rng = rng_for("torch_rs")
    x_np = rng.standard_normal(shape).astype(np.float32)
    w_np = rng.standard_normal(tuple(reversed(shape))).astype(np.float32)
    perm = tuple(reversed(range(len(shape))))
    x = torch_rs.tensor(x_np, device="cuda", requires_grad=True)
    w = torch_rs.tensor(w_np, device="cuda", requires_grad=True)
    wt = w.permute(*perm)
    p = x * wt
    r = p.relu()
    loss = r.sum()
    loss.backward()
    wt_np = np.transpose(w_np, perm)
    p_np = x_np * wt_np
    assert_bitwise_equal(p.numpy().reshape(-1), p_np.reshape(-1))
    g = (p_np > 0).astype(np.float32)  # relu': up where the input is positive (no NaNs here)
    assert_bitwise_equal(x.grad.numpy().reshape(-1), (g * wt_np).reshape(-1))
    gw = np.transpose(g * x_np, perm)
    assert_bitwise_equal(w.grad.numpy().reshape(-1), gw.reshape(-1))
    assert tuple(x.grad.shape) == shape


# ---- random layouts at ranks 6-14 -----------------------------------------

def _rand_shape(rng, rank, cap=200_000):
    while True:
        shape = tuple(int(rng.choice([1, 2, 2, 3])) for _ in range(rank))
        if np.prod(shape) <= cap:
            return shape


def _rand_strides(rng, shape):
    """A random physical dim order, inner stride 1 or 2, gaps between dims."""
    perm = rng.permutation(len(shape))
    strides = [0] * len(shape)
    step = int(rng.integers(1, 3))
    for d in reversed(perm):
        strides[d] = step
        step *= max(shape[d], 1) + int(rng.integers(0, 2))
    return tuple(strides)


def _rand_bshape(rng, oshape):
    rank = int(rng.integers(0, len(oshape) + 1))
    return tuple(1 if rng.random() < 0.3 else d for d in oshape[len(oshape) - rank:])


def _rand_view(rng, shape):
    st = _rand_strides(rng, shape)
    off = int(rng.integers(0, 3))
    return U.special_mix(rng, max(O.storage_size(shape, st, off), 1)), shape, st, off


@pytest.mark.parametrize("op", [O.ADD, O.MUL])
def test_random_high_rank_layouts_binary(op):
    """60 random layouts per op at ranks 6-14 (permuted dims with gaps,
    offsets, size-1 and broadcast dims): with or without a split, every
    kernel variant agrees with the oracle bit for bit."""
    rng = np.random.default_rng(9100 + op)
    for case in range(60):
        oshape = _rand_shape(rng, int(rng.integers(6, 15)))
        ash = oshape if rng.random() < 0.5 else _rand_bshape(rng, oshape)
        bsh = _rand_bshape(rng, oshape)
        a, ash, ast, aoff = _rand_view(rng, ash)
        b, bsh, bst, boff = _rand_view(rng, bsh)
        osh, ostr = O.binary_output_layout(ash, ast, bsh, bst)
        want = O.binary(op, a, ash, ast, aoff, b, bsh, bst, boff, osh, ostr)
        got = U.binary(op, a, ash, ast, aoff, b, bsh, bst, boff, osh, ostr)
        try:
            assert_bitwise_equal(got, want)
        except AssertionError as e:
            raise AssertionError(f"case {case}: a {ash} {ast} +{aoff}, b {bsh} {bst} +{boff}: {e}") from None


def test_random_high_rank_layouts_unary():
    rng = np.random.default_rng(9200)
    for case in range(60):
        shape = _rand_shape(rng, int(rng.integers(6, 15)))
        a, sh, st, off = _rand_view(rng, shape)
        ostr = O.unary_output_strides(sh, st)
        for op in (O.RELU, O.COPY):
            try:
                assert_bitwise_equal(U.unary(op, a, sh, st, off, ostr), O.unary(op, a, sh, st, off, ostr),
                                     nan_equal=False)
            except AssertionError as e:
                raise AssertionError(f"case {case} op {op}: {sh} {st} +{off}: {e}") from None


def test_random_high_rank_broadcast_reduction():
    """60 random (output, other, self) shapes at ranks 6-12: the multiply VJP
    accumulates in the reference's order bit for bit."""
    rng = np.random.default_rng(9300)
    for case in range(60):
        oshape = _rand_shape(rng, int(rng.integers(6, 13)), cap=100_000)
        self_shape = _rand_bshape(rng, oshape)
        oth_shape = _rand_bshape(rng, oshape) if rng.random() < 0.6 else oshape
        oth_strides = _rand_strides(rng, oth_shape)
        n = int(np.prod(oshape))
        up = U.special_mix(rng, n)
        other = U.special_mix(rng, max(O.storage_size(oth_shape, oth_strides, 0), 1))
        rc, got = gpu_mul_backward(up, oshape, other, oth_shape, oth_strides, self_shape)
        check(rc)
        want = O.mul_backward(up, oshape, other, oth_shape, oth_strides, 0, self_shape)
        try:
            assert_bitwise_equal(got, want)
        except AssertionError as e:
            raise AssertionError(f"case {case}: out {oshape}, other {oth_shape} {oth_strides}, "
                                 f"self {self_shape}: {e}") from None


def test_fused_transposing_roles_inside_a_split_launch():
    """(a + b) * c at rank 9 with c transposed in its last two dims and
    reversed in the outer ones, b broadcast over every outer dim (held in
    registers across a walk) and a constant along the transposed dim (loaded
    once per tuple): the inner 8 dims run the transposing kernel with its
    roles, once per index of the split dim, bit-exact against the oracle."""
    outer = (2, 3, 2, 3, 2, 3, 2)
    m, k = 64, 128
    shape = outer + (m, k)
    rng = rng_for("xpose_split")
    ashape = outer + (1, k)
    bshape = (1,) * len(outer) + (m, k)
    n = int(np.prod(shape))
    a = U.special_mix(rng, int(np.prod(ashape)))
    b = U.special_mix(rng, m * k)
    c = U.special_mix(rng, n)
    ast, bst = O.contiguous_strides(ashape), O.contiguous_strides(bshape)
    # c: a contiguous buffer laid out as reversed(outer) + (k, m), viewed in
    # outer + (m, k) order
    base = O.contiguous_strides(tuple(reversed(outer)) + (k, m))
    cst = tuple(reversed(base[:len(outer)])) + (1, m)
    lays = [layout_of(ashape, ast), layout_of(bshape, bst), layout_of(shape, cst)]
    info = abi.pointwise_plan(lays, layout_of(shape), roles=True)
    assert (info.variant, info.split, info.rank) == (3, 1, 8)  # transposing kernel, one split dim
    assert (info.trans, info.held, info.once) == (0b100, 0b010, 0b001)
    kid = U.fusion_compile("in f32\nin f32\nin f32\nadd %0 %1\nmul %3 %2\nout %4\n")
    out = U.out_buffer(n)
    U.fusion_launch(kid, [U.dev(a), U.dev(b), U.dev(c)], lays, out, layout_of(shape))
    ost = O.contiguous_strides(shape)
    t = O.binary(O.ADD, a, ashape, ast, 0, b, bshape, bst, 0, shape, ost)
    want = O.binary(O.MUL, t, shape, ost, 0, c, shape, cst, 0, shape, ost)
    assert_bitwise_equal(out.to_numpy(count=n), want)
    # the eager launcher plans the same layout without roles
    got = U.binary(O.MUL, t, shape, ost, 0, c, shape, cst, 0, shape, ost)
    assert_bitwise_equal(got, want)
