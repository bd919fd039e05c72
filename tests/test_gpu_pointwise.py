"""GPU parity of the eager pointwise entry points against the CPU oracle.

Bar: bit-exact for add/sub/mul/div, scalar ops, relu, neg, copy and
mask-apply (NaN payloads may differ by ISA, so any NaN equals any NaN except
where the reference fixes the result, e.g. relu(NaN) = +0.0); exp within
2 ulp of glibc expf.  Layouts cover contiguous, broadcast, transposed,
permuted, offset, unaligned, strided, scalar and empty operands.
"""
import ctypes
import zlib

import numpy as np
import pytest

import gpu_util as U
import oracle as O
from helpers import assert_bitwise_equal, check_bits, f32_from_bits, golden, ulp_distance
from trs_backend import abi

pytestmark = pytest.mark.gpu
G = golden()


def _view(rng, shape, strides=None, offset=0, storage=None):
    """A random storage plus a (shape, strides, offset) view into it."""
    if strides is None:
        strides = O.contiguous_strides(shape)
    need = max(O.storage_size(shape, strides, offset), 1)
    n = need if storage is None else storage
    return U.special_mix(rng, n), tuple(shape), tuple(strides), offset


def _transposed(rng, shape2):
    """A .T view of a contiguous matrix: logical shape (c, r), strides (1, c)."""
    r, c = shape2
    buf = U.special_mix(rng, r * c)
    return buf, (c, r), (1, c), 0


BINARY_CASES = {
    "flat_aligned": lambda rng: (_view(rng, (4096,)), _view(rng, (4096,))),
    "flat_tail": lambda rng: (_view(rng, (1001,)), _view(rng, (1001,))),
    "merged_2d": lambda rng: (_view(rng, (37, 129)), _view(rng, (37, 129))),
    "row_broadcast": lambda rng: (_view(rng, (64, 256)), _view(rng, (256,))),
    "row_broadcast_odd": lambda rng: (_view(rng, (33, 37)), _view(rng, (37,))),
    "row_broadcast_left": lambda rng: (_view(rng, (256,)), _view(rng, (64, 256))),
    "column_broadcast": lambda rng: (_view(rng, (64, 256)), _view(rng, (64, 1))),
    "mixed_ranks": lambda rng: (_view(rng, (2, 1, 3)), _view(rng, (3, 1))),
    "outer_broadcast": lambda rng: (_view(rng, (4, 1, 64)), _view(rng, (1, 32, 64))),
    "transposed_left": lambda rng: (_transposed(rng, (96, 80)), _view(rng, (80, 96))),
    "transposed_right": lambda rng: (_view(rng, (80, 96)), _transposed(rng, (96, 80))),
    "both_transposed": lambda rng: (_transposed(rng, (70, 50)), _transposed(rng, (70, 50))),
    "matrix_T_batched": lambda rng: (_view(rng, (4, 32, 64)), _view(rng, (4, 32, 64), (2048, 1, 32))),
    "offset_unaligned": lambda rng: (_view(rng, (33, 64), offset=1), _view(rng, (33, 64), offset=3)),
    "strided_gather": lambda rng: (_view(rng, (500,), (3,)), _view(rng, (500,), (2,), 1)),
    "rank0_left": lambda rng: (_view(rng, ()), _view(rng, (5, 7))),
    "rank0_right": lambda rng: (_view(rng, (5, 7)), _view(rng, ())),
    "permuted_3d": lambda rng: (_view(rng, (16, 32, 8), (1, 128, 16)), _view(rng, (16, 32, 8))),
    "empty": lambda rng: (_view(rng, (0, 5)), _view(rng, (5,))),
    "large_transposed_ragged": lambda rng: (_transposed(rng, (1000, 999)), _view(rng, (999, 1000))),
    # broadcasts that merge to no lower rank: the fixed rank-4 rows kernel, and
    # rank 5 through the run-time decode
    "rank4_broadcast": lambda rng: (_view(rng, (3, 1, 5, 64)), _view(rng, (1, 4, 1, 64))),
    "rank4_broadcast_wide": lambda rng: (_view(rng, (8, 1, 16, 1024)), _view(rng, (1, 8, 1, 1024))),
    "rank4_broadcast_ragged": lambda rng: (_view(rng, (5, 1, 7, 2051)), _view(rng, (1, 3, 1, 2051))),
    "rank5_broadcast": lambda rng: (_view(rng, (2, 1, 3, 1, 64)), _view(rng, (1, 3, 1, 4, 64))),
    # rows tiles of one float4 per lane with a partial last tile: 64-lane
    # blocks when an input streams, 128-lane blocks when only the output does
    "rows_partial_tile": lambda rng: (_view(rng, (64, 260)), _view(rng, (260,))),
    "rows_write_only_partial": lambda rng: (_view(rng, (8, 1, 516)), _view(rng, (1, 16, 516))),
    # more tiles in one tuple than the GPU holds at once: diagonal tile order
    "skewed_transposed": lambda rng: (_view(rng, (4096, 4096)), _transposed(rng, (4096, 4096))),
    "skewed_transposed_ragged": lambda rng: (_transposed(rng, (4099, 4100)), _view(rng, (4100, 4099))),
}


@pytest.mark.parametrize("case", sorted(BINARY_CASES))
@pytest.mark.parametrize("op", [O.ADD, O.SUB, O.MUL, O.DIV])
def test_binary_bit_exact(case, op):
    rng = np.random.default_rng(zlib.crc32(case.encode()) + op)
    (a, ash, ast, aoff), (b, bsh, bst, boff) = BINARY_CASES[case](rng)
    oshape, ostr = O.binary_output_layout(ash, ast, bsh, bst)
    want = O.binary(op, a, ash, ast, aoff, b, bsh, bst, boff, oshape, ostr)
    got = U.binary(op, a, ash, ast, aoff, b, bsh, bst, boff, oshape, ostr)
    assert_bitwise_equal(got, want)


SCALAR_CASES = {
    "contiguous": ((257, 33), None, 0),
    "transposed": ((40, 30), (1, 40), 0),
    "offset": ((100,), (1,), 5),
    "strided": ((100,), (3,), 0),
    "rank0": ((), (), 0),
}


@pytest.mark.parametrize("case", sorted(SCALAR_CASES))
@pytest.mark.parametrize("op", [O.S_ADD, O.S_SUB, O.S_MUL, O.S_DIV, O.S_RSUB, O.S_RDIV])
def test_scalar_bit_exact(case, op):
    rng = np.random.default_rng(op * 7 + len(case))
    shape, strides, off = SCALAR_CASES[case]
    x, shape, strides, off = _view(rng, shape, strides, off)
    ostr = O.scalar_output_strides(shape, strides)
    for s in (1.0, -0.0, 3.5e-3, np.float32(1 / 0.9)):
        want = O.scalar(op, x, shape, strides, off, float(s), ostr)
        got = U.scalar(op, x, shape, strides, off, float(s), ostr)
        assert_bitwise_equal(got, want)


UNARY_CASES = {
    "contiguous": (((1 << 16) + 3,), None, 0),
    "matrix": ((64, 1024), None, 0),
    "transposed": ((96, 80), (1, 96), 0),
    "permuted": ((8, 16, 32), (1, 256, 8), 0),
    "offset_unaligned": ((1000,), (1,), 1),
    "strided": ((1000,), (2,), 0),
    "rank0": ((), (), 0),
    "empty": ((3, 0), None, 0),
}


@pytest.mark.parametrize("case", sorted(UNARY_CASES))
@pytest.mark.parametrize("op", [O.RELU, O.NEG, O.COPY])
def test_unary_bit_exact(case, op):
    rng = np.random.default_rng(op + 100)
    shape, strides, off = UNARY_CASES[case]
    x, shape, strides, off = _view(rng, shape, strides, off)
    ostr = O.unary_output_strides(shape, strides)
    want = O.unary(op, x, shape, strides, off, ostr)
    got = U.unary(op, x, shape, strides, off, ostr)
    # relu maps NaN to +0.0 and neg flips a NaN's sign bit: compare every bit.
    assert_bitwise_equal(got, want, nan_equal=(op == O.COPY))


@pytest.mark.parametrize("case", sorted(UNARY_CASES))
def test_exp_within_two_ulp(case):
    rng = np.random.default_rng(5)
    shape, strides, off = UNARY_CASES[case]
    x, shape, strides, off = _view(rng, shape, strides, off)
    with np.errstate(over="ignore"):
        x = (x * 20).astype(np.float32)
    ostr = O.unary_output_strides(shape, strides)
    want = O.unary(O.EXP, x, shape, strides, off, ostr)
    got = U.unary(O.EXP, x, shape, strides, off, ostr)
    assert (np.isnan(got) == np.isnan(want)).all()
    assert ulp_distance(got, want).max(initial=0) <= 2


def test_exp_sweep_over_finite_range_within_two_ulp():
    # Every 97th bit pattern below |x| < 104 (about 22M inputs), incl. subnormal outputs.
    bits = np.arange(0, 0x42D00000, 97, dtype=np.uint32)
    x = np.concatenate([bits.view(np.float32), -bits.view(np.float32)])
    want = O.unary_contig(O.EXP, x)
    got = U.unary(O.EXP, x, (x.size,), (1,), 0, (1,))
    d = ulp_distance(got, want)
    assert d.max() <= 2, (x[d.argmax()], got[d.argmax()], want[d.argmax()])


def test_golden_relu_bits_on_gpu():
    g = G["relu_bits"]
    storage = np.concatenate([np.full(12, 1.0, np.float32), f32_from_bits(g["input_bits"])])
    v = g["offset_view"]
    out = U.unary(O.RELU, storage, v["shape"], v["strides"], v["offset"], v["out_strides"])
    check_bits(out, g["expected_bits"])
    t = g["transposed_view"]
    out = U.unary(O.RELU, storage, t["shape"], t["strides"], t["offset"], t["out_strides"])
    check_bits(np.array([out[i + 4 * j] for i in range(4) for j in range(3)], np.float32),
               g["transposed_expected_bits"])


@pytest.mark.parametrize("key,op", [("sub_nonfinite", O.SUB), ("div_nonfinite", O.DIV)])
def test_golden_nonfinite_on_gpu(key, op):
    g = G[key]
    n = len(g["left"])
    out = U.binary(op, f32_from_bits(g["left"]), (n,), (1,), 0, f32_from_bits(g["right"]), (n,), (1,), 0, (n,), (1,))
    check_bits(out, g["expected"])


@pytest.mark.parametrize("op,s,key", [
    (O.S_ADD, 2.0, "add_scalar_2"), (O.S_SUB, 2.0, "sub_scalar_2"), (O.S_RSUB, 2.0, "scalar_sub_2"),
    (O.S_MUL, 2.0, "mul_scalar_2"), (O.S_DIV, -0.0, "div_scalar_neg0"), (O.S_RDIV, -0.0, "scalar_div_neg0")])
def test_golden_scalar_signed_zero_on_gpu(op, s, key):
    g = G["scalar_signed_zero"]
    out = U.scalar(op, np.array(g["input"], np.float32), (4,), (1,), 0, s, (1,))
    check_bits(out, g[key])


def test_golden_scalar_div_reciprocal_on_gpu():
    g = G["scalar_div_reciprocal"]
    out = U.scalar(O.S_RDIV, f32_from_bits([g["denominator_bits"]]), (1,), (1,), 0,
                   float(f32_from_bits([g["scalar_bits"]])[0]), (1,))
    check_bits(out, [g["expected_bits"]])


@pytest.mark.parametrize("op,key", [(O.ADD, "add"), (O.SUB, "sub"), (O.MUL, "mul"), (O.DIV, "div")])
def test_golden_broadcast_mixed_ranks_on_gpu(op, key):
    g = G["broadcast_mixed_ranks"]
    ls, rs = g["left_shape"], g["right_shape"]
    oshape, ostr = O.binary_output_layout(ls, O.contiguous_strides(ls), rs, O.contiguous_strides(rs))
    out = U.binary(op, np.array(g["left"], np.float32), ls, O.contiguous_strides(ls), 0,
                   np.array(g["right"], np.float32), rs, O.contiguous_strides(rs), 0, oshape, ostr)
    assert out.tolist() == g[key]


@pytest.mark.parametrize("shape,mshape", [((8192,), (8192,)), ((64, 1000), (64, 1000)), ((3, 5), (3, 5))])
def test_mask_apply_bit_exact(shape, mshape):
    rng = np.random.default_rng(21)
    n = int(np.prod(shape))
    h = U.special_mix(rng, n)
    mask = (rng.random(n) < 0.9).astype(np.uint8)
    scale = np.float32(1 / 0.9)
    want = O.mask_apply(h, mask, float(scale))
    dh, dm = U.dev(h), U.dev(mask)
    do = U.out_buffer(n)
    lay = abi.layout_of(shape)
    abi.check(abi.lib.trs_mask_apply_f32(dh.ptr, ctypes.byref(lay), dm.ptr, ctypes.byref(abi.layout_of(mshape)),
                                         ctypes.c_float(scale), do.ptr, ctypes.byref(lay)))
    assert_bitwise_equal(do.to_numpy(count=n), want)


def test_shape_mismatch_is_an_error_not_a_launch():
    a = U.dev(np.zeros(4, np.float32))
    out = U.out_buffer(4)
    rc = abi.lib.trs_binary_f32(O.ADD, a.ptr, ctypes.byref(abi.layout_of((2, 2))), a.ptr,
                                ctypes.byref(abi.layout_of((4,))), out.ptr, ctypes.byref(abi.layout_of((2, 2))))
    assert rc == -4
    assert "must match the size of tensor" in abi.lib.trs_last_error().decode()


def _random_layout_view(rng, shape):
    """A view of `shape` with a random physical dim order, inner stride 1 or
    2, random gaps between dims and a random offset."""
    r = len(shape)
    perm = rng.permutation(r)
    strides = [0] * r
    step = int(rng.integers(1, 3))
    for d in reversed(perm):
        strides[d] = step
        step *= max(shape[d], 1) + int(rng.integers(0, 2))
    return _view(rng, shape, strides, int(rng.integers(0, 3)))


def _random_broadcast_shape(rng, oshape):
    """A right-aligned operand shape that broadcasts to oshape."""
    rank = int(rng.integers(0, len(oshape) + 1))
    return tuple(1 if rng.random() < 0.3 else d for d in oshape[len(oshape) - rank:])


@pytest.mark.parametrize("op", [O.ADD, O.SUB, O.MUL, O.DIV])
def test_random_layouts_binary_bit_exact(op):
    """150 random layouts per op (rank 1-5, size-1 and broadcast dims,
    permuted strides with gaps, offsets): the host planner's dim dropping,
    ordering and merging plus every kernel variant agree with the oracle bit
    for bit."""
    rng = np.random.default_rng(4242 + op)
    for case in range(150):
        rank = int(rng.integers(1, 6))
        oshape = tuple(int(rng.choice([1, 2, 3, 5, 8, 17])) for _ in range(rank))
        ash, bsh = _random_broadcast_shape(rng, oshape), _random_broadcast_shape(rng, oshape)
        if rng.random() < 0.5:
            ash = oshape
        a, ash, ast, aoff = _random_layout_view(rng, ash)
        b, bsh, bst, boff = _random_layout_view(rng, bsh)
        osh, ostr = O.binary_output_layout(ash, ast, bsh, bst)
        want = O.binary(op, a, ash, ast, aoff, b, bsh, bst, boff, osh, ostr)
        got = U.binary(op, a, ash, ast, aoff, b, bsh, bst, boff, osh, ostr)
        try:
            assert_bitwise_equal(got, want)
        except AssertionError as e:
            raise AssertionError(f"case {case}: a {ash} {ast} +{aoff}, b {bsh} {bst} +{boff}: {e}") from None


@pytest.mark.parametrize("op", [O.RELU, O.NEG])
def test_random_layouts_unary_bit_exact(op):
    rng = np.random.default_rng(777 + op)
    for case in range(150):
        rank = int(rng.integers(0, 6))
        shape = tuple(int(rng.choice([1, 2, 3, 5, 8, 17])) for _ in range(rank))
        a, sh, st, off = _random_layout_view(rng, shape) if rank else _view(rng, ())
        ostr = O.unary_output_strides(sh, st)
        want = O.unary(op, a, sh, st, off, ostr)
        got = U.unary(op, a, sh, st, off, ostr)
        try:
            assert_bitwise_equal(got, want, nan_equal=False)  # relu and neg are exact on NaNs too
        except AssertionError as e:
            raise AssertionError(f"case {case}: {sh} {st} +{off}: {e}") from None


def _random_big_view(rng, shape, perm):
    """A view of `shape` whose dims lie in memory in the order `perm`
    (outermost first), unit inner stride, sometimes a padded row, and an
    offset of 0, 4 (aligned) or 1 (unaligned)."""
    r = len(shape)
    strides = [0] * r
    step = 1
    for d in reversed(perm):
        strides[d] = step
        step *= max(shape[d], 1) + (4 if rng.random() < 0.2 else 0)
    return _view(rng, shape, strides, int(rng.choice([0, 0, 4, 1])))


@pytest.mark.parametrize("op", [O.ADD, O.MUL])
def test_random_large_layouts_binary_bit_exact(op):
    """40 random layouts per op at sizes the kernels' fast cases and edge
    paths need (rank 2-4, dims up to 4100, up to 16M elements): transposed
    and permuted operands, broadcasts, padded rows, aligned and unaligned
    offsets, so the fixed-rank rows kernels, the transposing kernel in both
    tile orders and the ragged tiles are all checked against the oracle."""
    rng = np.random.default_rng(90210 + op)
    dims = [1, 2, 5, 64, 129, 1024, 2048, 4096, 4100]
    for case in range(40):
        rank = int(rng.integers(2, 5))
        while True:
            oshape = tuple(int(rng.choice(dims)) for _ in range(rank))
            if 1 << 16 <= int(np.prod(oshape)) <= 1 << 24:
                break
        ash, bsh = _random_broadcast_shape(rng, oshape), _random_broadcast_shape(rng, oshape)
        if rng.random() < 0.6:
            ash = oshape
        # operand dims in memory order: b's reverses a's half the time (a
        # transpose between them), else each is plain or randomly permuted
        pa = rng.permutation(len(ash)) if rng.random() < 0.3 else np.arange(len(ash))
        if rng.random() < 0.5 and len(bsh) == len(ash):
            pb = pa[::-1]
        else:
            pb = rng.permutation(len(bsh)) if rng.random() < 0.3 else np.arange(len(bsh))
        a, ash, ast, aoff = _random_big_view(rng, ash, pa)
        b, bsh, bst, boff = _random_big_view(rng, bsh, pb)
        osh, ostr = O.binary_output_layout(ash, ast, bsh, bst)
        want = O.binary(op, a, ash, ast, aoff, b, bsh, bst, boff, osh, ostr)
        got = U.binary(op, a, ash, ast, aoff, b, bsh, bst, boff, osh, ostr)
        try:
            assert_bitwise_equal(got, want)
        except AssertionError as e:
            raise AssertionError(f"case {case}: a {ash} {ast} +{aoff}, b {bsh} {bst} +{boff}: {e}") from None


def test_reference_fast_path_vectors_on_gpu():
    """The operands of src/tensor.rs:4887-5024 (signalling NaNs, infinities,
    signed zeros and denormals; an offset transposed view, a rank-mixing
    broadcast, a row view and an offset rank-0 NaN) through every binary op:
    the planner's output strides, including [1, 3] for strided + row
    (src/tensor.rs:5015), and values bit-exact against the oracle (any NaN
    equals any NaN, as the payload is the ISA's)."""
    def strided(bits):  # offset_strided_matrix (src/tensor.rs:4700-4709)
        return (np.concatenate([np.zeros(9, np.float32), f32_from_bits(bits)]), (3, 3), (1, 3), 9)

    left = strided([0x7F812345, 0xFFC54321, 0x7F800000, 0xFF800000, 0x0, 0x80000000, 0x1, 0x80000001, 0x3F800000])
    right = strided([0xFF854321, 0x7FC12345, 0xFF800000, 0x7F800000, 0x80000000, 0x0, 0x80000001, 0x1, 0xBF800000])
    bcast_l = (f32_from_bits([0x7F812345, 0xFFC54321, 0x7F800000, 0xFF800000, 0x0, 0x80000000]), (2, 1, 3), (3, 3, 1), 0)
    bcast_r = (f32_from_bits([0xFF854321, 0x80000001]), (1, 2, 1), (2, 1, 1), 0)
    row = (f32_from_bits([0, 0, 0, 0xFF854321, 0x80000001, 0xBF800000]), (3,), (1,), 3)
    nan_scalar = (f32_from_bits([0, 0xFF812345]), (), (), 1)
    pairs = [(left, right), (bcast_l, bcast_r), (left, row), (nan_scalar, left), (left, nan_scalar)]
    assert O.binary_output_layout(left[1], left[2], row[1], row[2])[1] == (1, 3)
    for (a, ash, ast, aoff), (b, bsh, bst, boff) in pairs:
        osh, ostr = O.binary_output_layout(ash, ast, bsh, bst)
        for op in (O.ADD, O.SUB, O.MUL, O.DIV):
            want = O.binary(op, a, ash, ast, aoff, b, bsh, bst, boff, osh, ostr)
            got = U.binary(op, a, ash, ast, aoff, b, bsh, bst, boff, osh, ostr)
            assert_bitwise_equal(got, want)
