"""GPU parity of the reduction and backward entry points against the oracle.

relu VJP, Multiply VJP (with and without broadcast), the add VJP
(reduce-to-shape), accumulation and fills are bit-exact: the device kernels
keep the reference's per-element expressions and its output-major
accumulation order.  sum uses a fixed-order tree, checked within the tree's
own depth bound against the exact sum, exact on small integers, and with the
reference's -0.0 start value.
"""
import ctypes

import numpy as np
import pytest

import gpu_util as U
import oracle as O
from helpers import assert_bitwise_equal, check_bits, f32_from_bits, golden
from trs_backend import abi
from trs_backend.abi import check, layout_of

pytestmark = pytest.mark.gpu
G = golden()


def gpu_relu_backward(x, shape, strides, off, up):
    dx, du = U.dev(x), U.dev(up)
    n = int(np.prod(shape)) if shape else 1
    do = U.out_buffer(n)
    check(abi.lib.trs_relu_backward_f32(dx.ptr, ctypes.byref(layout_of(shape, strides, off)), du.ptr, do.ptr))
    return do.to_numpy(count=n)


def gpu_mul_backward(up, oshape, other, oth_shape, oth_strides, oth_off, self_shape):
    du, dother = U.dev(up), U.dev(other)
    n = int(np.prod(self_shape)) if self_shape else 1
    do = U.out_buffer(n)
    check(abi.lib.trs_mul_backward_f32(du.ptr, ctypes.byref(layout_of(oshape)), dother.ptr,
                                       ctypes.byref(layout_of(oth_shape, oth_strides, oth_off)),
                                       ctypes.byref(layout_of(self_shape)), do.ptr))
    return do.to_numpy(count=n)


def gpu_reduce(up, oshape, self_shape):
    du = U.dev(up)
    n = int(np.prod(self_shape)) if self_shape else 1
    do = U.out_buffer(n)
    check(abi.lib.trs_reduce_to_shape_f32(du.ptr, ctypes.byref(layout_of(oshape)), ctypes.byref(layout_of(self_shape)),
                                          do.ptr))
    return do.to_numpy(count=n)


def gpu_sum(x, shape, strides=None, off=0):
    dx = U.dev(x)
    do = U.out_buffer(1)
    check(abi.lib.trs_sum_f32(dx.ptr, ctypes.byref(layout_of(shape, strides, off)), do.ptr))
    return do.to_numpy(count=1)[0]


def test_relu_vjp_golden_bits():
    g = G["autograd_relu_vjp"]
    x = f32_from_bits(g["input_bits"])
    w = f32_from_bits(g["weight_bits"])
    n = x.size
    up_relu = gpu_mul_backward(np.ones(n, np.float32), (n,), w, (n,), (1,), 0, (n,))
    grad = gpu_relu_backward(x, (n,), (1,), 0, up_relu)
    check_bits(grad, g["expected_gradient_bits"])


@pytest.mark.parametrize("shape,strides,off", [((4096,), (1,), 0), ((64, 96), (1, 64), 0), ((300,), (2,), 1),
                                               ((8, 16, 32), (1, 256, 8), 0), ((), (), 0)])
def test_relu_vjp_layouts(shape, strides, off):
    rng = np.random.default_rng(1)
    need = O.storage_size(shape, strides, off)
    x = U.special_mix(rng, max(need, 1))
    n = int(np.prod(shape)) if shape else 1
    up = U.special_mix(rng, n)
    assert_bitwise_equal(gpu_relu_backward(x, shape, strides, off, up), O.relu_backward(x, shape, strides, off, up),
                         nan_equal=False)


MUL_CASES = [
    # (out shape, other shape, other strides, self shape)
    ((4096,), (4096,), (1,), (4096,)),
    ((64, 96), (64, 96), (96, 1), (64, 96)),
    ((64, 96), (96,), (1,), (64, 96)),          # other broadcast, self full: stored as is
    ((64, 96), (64, 96), (96, 1), (96,)),       # self broadcast over rows
    ((64, 96), (64, 96), (96, 1), (64, 1)),     # self broadcast over columns
    ((2, 3), (1, 3), (3, 1), (2, 1)),           # autograd.rs:176-188
    ((4, 5, 6), (4, 5, 6), (30, 6, 1), ()),     # rank-0 operand
    ((4, 5, 6), (5, 1), (1, 1), (4, 1, 6)),
    ((3, 2), (3, 2), (1, 3), ()),               # transposed other
    ((0, 3), (0, 3), (3, 1), (3,)),             # empty output
]


@pytest.mark.parametrize("case", MUL_CASES, ids=[str(c) for c in MUL_CASES])
def test_mul_vjp_bit_exact(case):
    oshape, oth_shape, oth_strides, self_shape = case
    rng = np.random.default_rng(len(oshape) * 31 + sum(oshape))
    n = int(np.prod(oshape))
    up = U.special_mix(rng, max(n, 1))[:n] if n else np.zeros(0, np.float32)
    other = U.special_mix(rng, max(O.storage_size(oth_shape, oth_strides), 1))
    want = O.mul_backward(up if n else np.zeros(1, np.float32), oshape, other, oth_shape, oth_strides, 0, self_shape)
    got = gpu_mul_backward(up if n else np.zeros(1, np.float32), oshape, other, oth_shape, oth_strides, 0,
                           self_shape)
    assert_bitwise_equal(got, want)


def test_mul_vjp_negative_zero_rules():
    g = G["autograd_negative_zero"]
    nb = g["no_broadcast"]
    got = gpu_mul_backward(np.ones(1, np.float32), (1,), f32_from_bits(nb["right_bits"]), (1,), (1,), 0, (1,))
    check_bits(got, nb["left_grad_bits"])
    b = g["broadcast"]
    got = gpu_mul_backward(np.ones(2, np.float32), (2,), f32_from_bits(b["right_bits"]), (2,), (1,), 0, ())
    check_bits(got, b["left_grad_bits"])


@pytest.mark.parametrize("oshape,self_shape", [((8192, 1024), (1024,)), ((64, 96), (64, 1)), ((4, 5, 6), (5, 1)),
                                               ((4, 5, 6), ()), ((7, 9), (7, 9))])
def test_add_vjp_reduce_to_shape_bit_exact(oshape, self_shape):
    rng = np.random.default_rng(2)
    up = rng.standard_normal(int(np.prod(oshape))).astype(np.float32)
    assert_bitwise_equal(gpu_reduce(up, oshape, self_shape), O.reduce_to_shape(up, oshape, self_shape))


# Shapes that take the staged reduction (the reduced dims merge into at least
# one 256-row stage, the kept inner part is a multiple of 32 chains): the bias
# gradient of the MLP, config 2's `a` operand, a partial last stage, a single
# stage, outer kept dims, a reduced dim between kept ones, 32 chains only, and
# a row count that is not a multiple of 4.
STAGED = [((8192, 4096), (4096,)), ((8192, 1024), (1024,)), ((64, 512, 1024), (64, 1, 1024)),
          ((300, 128), (128,)), ((256, 64), (64,)), ((3, 1000, 192), (3, 1, 192)), ((2, 258, 96), (2, 1, 96)),
          ((2, 700, 5, 128), (2, 1, 5, 128)), ((1030, 2, 64), (2, 64)), ((4099, 32), (32,))]


@pytest.mark.parametrize("oshape,self_shape", STAGED)
def test_staged_reduce_to_shape_bit_exact(oshape, self_shape):
    """The add VJP through the staged kernel: every chain added in the
    reference's row-major order from +0.0, bit for bit."""
    rng = np.random.default_rng(sum(oshape))
    up = rng.standard_normal(int(np.prod(oshape))).astype(np.float32)
    up[::977] = -0.0
    assert_bitwise_equal(gpu_reduce(up, oshape, self_shape), O.reduce_to_shape(up, oshape, self_shape))


@pytest.mark.parametrize("oshape,self_shape", STAGED[:7])
@pytest.mark.parametrize("transposed", [False, True])
def test_staged_mul_vjp_bit_exact(oshape, self_shape, transposed):
    """The Multiply VJP of a broadcast operand through the staged kernel:
    contributions up*other (one rounding) added in order; `other` contiguous
    (vectors of 4 chains) or a transposed view of its last two dims, as c.mT
    in config 2 (vectors of 4 rows; one float at a time when the row count
    or the chain stride is not a multiple of 4)."""
    rng = np.random.default_rng(7 * sum(oshape) + transposed)
    n = int(np.prod(oshape))
    up = rng.standard_normal(n).astype(np.float32)
    other = rng.standard_normal(n).astype(np.float32)
    if transposed and len(oshape) >= 2:
        *lead, m, k = oshape
        base = O.contiguous_strides(tuple(lead) + (k, m))
        ostr = tuple(base[:-2]) + (base[-1], base[-2])
    else:
        ostr = O.contiguous_strides(oshape)
    got = gpu_mul_backward(up, oshape, other, oshape, ostr, 0, self_shape)
    want = O.mul_backward(up, oshape, other, oshape, ostr, 0, self_shape)
    assert_bitwise_equal(got, want)


@pytest.mark.parametrize("oshape,other_shape", [((1024, 4096), (4096,)), ((2, 300, 64), (2, 1, 64))])
def test_staged_mul_vjp_other_broadcast_along_rows(oshape, other_shape):
    """other constant along the reduced rows (stride 0 there): the 4-chain
    vectors re-read one row of other for every row of up."""
    rng = np.random.default_rng(len(oshape))
    n = int(np.prod(oshape))
    up = rng.standard_normal(n).astype(np.float32)
    other = rng.standard_normal(int(np.prod(other_shape))).astype(np.float32)
    ostr = O.contiguous_strides(other_shape)
    self_shape = other_shape
    got = gpu_mul_backward(up, oshape, other, other_shape, ostr, 0, self_shape)
    assert_bitwise_equal(got, O.mul_backward(up, oshape, other, other_shape, ostr, 0, self_shape))


def test_staged_reduction_unaligned_input_takes_the_unrolled_kernel():
    """up at an odd float offset cannot be read as 16-byte vectors: the
    unrolled one-lane-per-chain kernel runs instead, with the same bits."""
    rng = np.random.default_rng(99)
    oshape, self_shape = (1024, 256), (256,)
    up = rng.standard_normal(1024 * 256 + 1).astype(np.float32)
    du = U.dev(up)
    do = U.out_buffer(256)
    # up starts one float into the buffer (4-byte, not 16-byte, aligned)
    check(abi.lib.trs_reduce_to_shape_f32(ctypes.c_void_p(du.addr + 4), ctypes.byref(layout_of(oshape)),
                                          ctypes.byref(layout_of(self_shape)), do.ptr))
    assert_bitwise_equal(do.to_numpy(count=256), O.reduce_to_shape(up[1:], oshape, self_shape))


def sum_tree_depth(n: int) -> int:
    """Most roundings any element passes through in trs_sum_f32's fixed tree:
    one block (n <= 32768) adds ceil(n/256) terms per lane, then 8 tree
    levels; above that each of at most 1024 blocks adds ceil(chunk/256) per
    lane and 8 levels, and pass 2 adds 4 partials per lane and 8 levels."""
    if n <= 32768:
        return -(-n // 256) + 8
    chunk = -(-n // 1024)
    return -(-chunk // 256) + 8 + 4 + 8


@pytest.mark.parametrize("n", [1, 3, 1000, 32768, 32769, 1 << 20, (1 << 23) + 5])
@pytest.mark.parametrize("dist", ["normal", "positive"])
def test_sum_within_its_tree_bound(n, dist):
    """|device - exact| <= d * 2^-24 * sum|x| with d the tree's depth (52 at
    the MLP loss's 2^23 elements, against 2^24 for a sequential fold), the
    exact sum taken with math.fsum over the float64 values.  Positive data
    (no cancellation) makes a dropped or doubled block show as a gross error.
    The sequential oracle fold is compared within the sum of both bounds."""
    import math
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n) if dist == "normal" else rng.uniform(0.5, 1.5, n)
    x = x.astype(np.float32)
    got = float(gpu_sum(x, (n,)))
    exact = math.fsum(x.astype(np.float64))
    abs_sum = O.sum_abs(x)
    d = sum_tree_depth(n)

    def gamma(k):  # Higham's gamma_k = k u / (1 - k u), u = 2^-24
        return k * 2.0 ** -24 / (1 - k * 2.0 ** -24)

    assert abs(got - exact) <= gamma(d) * abs_sum, (got, exact, d)
    want = float(O.sum_f32(x, (n,)))
    assert abs(want - exact) <= gamma(n - 1) * abs_sum
    assert abs(got - want) <= (gamma(d) + gamma(n - 1)) * abs_sum


def device_tree_sum(x: np.ndarray) -> np.float32:
    """trs_sum_f32's documented order in float32 numpy (one rounding per add):
    a block over a contiguous range has 256 lanes; lane l adds elements l,
    l+256, ... of the range in order from -0.0, then the lanes meet in a tree
    (lane i += lane i+w for w = 128, 64, ..., 1).  Up to 32768 elements one
    block covers all; above, block b covers [b*chunk, (b+1)*chunk) with chunk =
    ceil(n/1024), and one more block sums the partials the same way."""
    def block(vals):
        acc = np.full(256, -0.0, np.float32)
        for s in range(0, vals.size, 256):
            seg = vals[s:s + 256]
            acc[:seg.size] = acc[:seg.size] + seg
        w = 128
        while w:
            acc[:w] = acc[:w] + acc[w:2 * w]
            w >>= 1
        return acc[0]

    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    if x.size <= 32768:
        return block(x)
    chunk = -(-x.size // 1024)
    partial = np.array([block(x[b:b + chunk]) for b in range(0, x.size, chunk)], np.float32)
    return block(partial)


@pytest.mark.parametrize("n", [1, 255, 32768, 32769, 1 << 20, (1 << 23) + 5])
def test_sum_follows_its_documented_tree_bit_for_bit(n):
    """The device sum is the fixed tree its header documents, exactly: the
    kernel may reorder loads for speed but never additions."""
    rng = np.random.default_rng(n + 11)
    x = rng.standard_normal(n).astype(np.float32) * np.float32(1000.0)
    got = np.float32(gpu_sum(x, (n,)))
    assert got.view(np.uint32) == device_tree_sum(x).view(np.uint32)
    if n >= 1000:  # a transposed view sums in logical order
        r = n // 37
        m = x[: r * 37].reshape(37, r)
        got = np.float32(gpu_sum(np.ascontiguousarray(m), (r, 37), (1, r)))
        assert got.view(np.uint32) == device_tree_sum(m.T).view(np.uint32)


@pytest.mark.parametrize("n", [1, 2, 257, 32768, 40000, 1 << 20])
def test_sum_of_negative_zeros_is_negative_zero(n):
    """Rust's f32 Sum starts from -0.0 (the oracle's fold does too): an
    all-(-0.0) input sums to -0.0 on the one-block and two-pass paths, while
    one +0.0 among them gives +0.0."""
    x = np.full(n, -0.0, np.float32)
    got = np.float32(gpu_sum(x, (n,)))
    want = O.sum_f32(x, (n,))
    assert got.view(np.uint32) == want.view(np.uint32) == 0x80000000
    x[n // 2] = 0.0
    got = np.float32(gpu_sum(x, (n,)))
    assert got.view(np.uint32) == O.sum_f32(x, (n,)).view(np.uint32) == 0


@pytest.mark.parametrize("n", [257, 32768, 32769, 100003])
def test_sum_of_small_integers_is_exact_on_both_paths(n):
    # Integers below 2^24 in total sum exactly in any order: the one-block
    # path (n <= 32768) and the two-pass path must both equal the fold.
    x = (np.arange(n) % 7 - 3).astype(np.float32)
    assert float(gpu_sum(x, (n,))) == float(O.sum_f32(x, (n,)))
    xt = x[: (n // 3) * 3].reshape(3, -1)
    got = gpu_sum(np.ascontiguousarray(xt), (xt.shape[1], 3), (1, xt.shape[1]))  # a transposed view
    assert float(got) == float(xt.sum())


def test_sum_of_transposed_view_and_golden():
    s = G["stride_aware_broadcast"]
    got = gpu_sum(np.arange(24, dtype=np.float32), s["shape"], s["strides"])
    assert int(np.float32(got).view(np.uint32)) == int(s["sum_bits"], 16)
    assert gpu_sum(np.array(G["sum_small"]["input"], np.float32), (3,)) == G["sum_small"]["expected"]


def test_accumulate_and_fill():
    rng = np.random.default_rng(3)
    a = rng.standard_normal(10001).astype(np.float32)
    b = rng.standard_normal(10001).astype(np.float32)
    da, db = U.dev(a), U.dev(b)
    check(abi.lib.trs_accumulate_f32(da.ptr, db.ptr, a.size))
    want = a.copy()
    O.lib().orc_accumulate_f32(want.ctypes.data, b.ctypes.data, a.size)
    assert_bitwise_equal(da.to_numpy(count=a.size), want)
    check(abi.lib.trs_fill_f32(da.ptr, 100, ctypes.c_float(-0.0)))
    assert (da.to_numpy(count=100).view(np.uint32) == 0x80000000).all()
    src = U.dev(np.array([2.5], np.float32))
    check(abi.lib.trs_fill_from_device_f32(da.ptr, 77, src.ptr))
    assert (da.to_numpy(count=77) == 2.5).all()


def _rand_bshape(rng, oshape):
    rank = int(rng.integers(0, len(oshape) + 1))
    return tuple(1 if rng.random() < 0.35 else d for d in oshape[len(oshape) - rank:])


def _rand_strides(rng, shape):
    r = len(shape)
    perm = rng.permutation(r)
    strides = [0] * r
    step = 1
    for d in reversed(perm):
        strides[d] = step
        step *= max(shape[d], 1) + int(rng.integers(0, 2))
    return tuple(strides)


def test_random_broadcast_mul_vjp_and_reduce_bit_exact():
    """150 random (output, other, self) broadcast shapes of rank 0-5 with the
    other operand in random layouts: the mul VJP and the add VJP's
    reduce_to_shape accumulate in the reference's order (from +0.0 over the
    reduced dims in output row-major order, or as-is with no broadcast) bit
    for bit."""
    rng = np.random.default_rng(515)
    for case in range(150):
        rank = int(rng.integers(0, 6))
        oshape = tuple(int(rng.choice([1, 2, 3, 4, 7, 9])) for _ in range(rank))
        self_shape = _rand_bshape(rng, oshape)
        oth_shape = _rand_bshape(rng, oshape) if rng.random() < 0.6 else oshape
        oth_strides = _rand_strides(rng, oth_shape)
        oth_off = int(rng.integers(0, 3))
        n = int(np.prod(oshape)) if oshape else 1
        up = U.special_mix(rng, max(n, 1))[:n]
        other = U.special_mix(rng, max(O.storage_size(oth_shape, oth_strides, oth_off), 1))
        try:
            want = O.mul_backward(up, oshape, other, oth_shape, oth_strides, oth_off, self_shape)
            got = gpu_mul_backward(up, oshape, other, oth_shape, oth_strides, oth_off, self_shape)
            assert_bitwise_equal(got, want)
            assert_bitwise_equal(gpu_reduce(up, oshape, self_shape), O.reduce_to_shape(up, oshape, self_shape))
        except AssertionError as e:
            raise AssertionError(f"case {case}: out {oshape}, other {oth_shape} {oth_strides} +{oth_off}, "
                                 f"self {self_shape}: {e}") from None


@pytest.mark.parametrize("oshape,self_shape", [((4099, 32), (32,)), ((1030, 64), (64,)), ((2, 700, 96), (2, 1, 96))])
def test_staged_mul_vjp_scalar_other_reads_on_16_chain_blocks(oshape, self_shape):
    """Few chains over at least 512 rows take 16-chain blocks; `other`
    transposed with a row count that is not a multiple of 4 is read one
    float at a time.  Bit for bit against the oracle."""
    rng = np.random.default_rng(sum(oshape))
    n = int(np.prod(oshape))
    up = rng.standard_normal(n).astype(np.float32)
    other = rng.standard_normal(n).astype(np.float32)
    *lead, m, k = oshape
    base = O.contiguous_strides(tuple(lead) + (k, m))
    ostr = tuple(base[:-2]) + (base[-1], base[-2])
    got = gpu_mul_backward(up, oshape, other, oshape, ostr, 0, self_shape)
    assert_bitwise_equal(got, O.mul_backward(up, oshape, other, oshape, ostr, 0, self_shape))
