"""Pin the oracle where the reference tests leave it open, by mathematics.

Each check is chosen so that a plausible mistake in the restatement (a
dropped term, a transposed operand, a wrong accumulation order or start
value, a fused multiply-add) fails it.
"""
import numpy as np
import pytest

import oracle as O
from helpers import assert_bitwise_equal, ulp_distance


def _rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 2), (7, 4, 9), (16, 33, 5)])
def test_matmul_exact_on_small_integers(m, k, n):
    # Products and partial sums of small integers are exact in f32: any order,
    # any operand mistake shows up as a wrong integer.
    rng = _rng(m * 100 + k * 10 + n)
    a = rng.integers(-8, 9, size=(m, k)).astype(np.float32)
    b = rng.integers(-8, 9, size=(k, n)).astype(np.float32)
    got = O.matmul(a.ravel(), (m, k), (k, 1), 0, b.ravel(), (k, n), (n, 1), 0).reshape(m, n)
    assert np.array_equal(got, (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))
    # transposed-view operands give the same result
    got_t = O.matmul(np.ascontiguousarray(a.T).ravel(), (m, k), (1, m), 0,
                     np.ascontiguousarray(b.T).ravel(), (k, n), (1, k), 0).reshape(m, n)
    assert np.array_equal(got, got_t)


def test_matmul_sequential_order_without_fma():
    # The reference order is c = +0; c = c + a_k*b_k for k ascending, with the
    # product rounded before the add.  Recompute that recurrence with numpy
    # float32 scalars (which round each op) and demand bit equality.
    rng = _rng(7)
    m, k, n = 4, 37, 3
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    got = O.matmul(a.ravel(), (m, k), (k, 1), 0, b.ravel(), (k, n), (n, 1), 0).reshape(m, n)
    want = np.zeros((m, n), np.float32)
    for i in range(m):
        for j in range(n):
            c = np.float32(0.0)
            for t in range(k):
                c = np.float32(c + np.float32(a[i, t] * b[t, j]))
            want[i, j] = c
    assert_bitwise_equal(got, want)


def test_matmul_rows_and_batch_agree_with_full():
    rng = _rng(11)
    a = rng.standard_normal((3, 6, 5)).astype(np.float32)
    b = rng.standard_normal((3, 5, 4)).astype(np.float32)
    full = O.matmul(a.ravel(), (6, 5), (5, 1), 0, b.ravel(), (5, 4), (4, 1), 0, batch=3, bsa=30, bsb=20)
    full = full.reshape(3, 6, 4)
    for t in range(3):
        single = O.matmul(a[t].ravel(), (6, 5), (5, 1), 0, b[t].ravel(), (5, 4), (4, 1), 0).reshape(6, 4)
        assert_bitwise_equal(full[t], single)
    rows, bound = O.matmul_rows(a[1].ravel(), (6, 5), (5, 1), b[1].ravel(), (5, 4), (4, 1), [0, 5, 2])
    assert_bitwise_equal(rows, full[1][[0, 5, 2]])
    assert np.allclose(bound, np.abs(a[1][[0, 5, 2]]).astype(np.float64) @ np.abs(b[1]).astype(np.float64))


def test_exp_is_within_one_ulp_of_correct_rounding():
    # glibc expf is documented < 1 ulp; check against exp in float64 rounded.
    rng = _rng(3)
    x = np.concatenate([rng.uniform(-103.0, 88.7, 200_000), rng.uniform(-1, 1, 50_000)]).astype(np.float32)
    got = O.unary_contig(O.EXP, x)
    want = np.exp(x.astype(np.float64)).astype(np.float32)
    assert ulp_distance(got, want).max() <= 1


def test_relu_exhaustive_sample_matches_closed_form():
    # relu_value: exact zeros kept (incl. -0.0), NaN -> +0.0, else max(v, 0).
    rng = _rng(5)
    bits = rng.integers(0, 2**32, size=1_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    got = O.unary_contig(O.RELU, x)
    want = np.where(x > 0, x, np.float32(0.0)).astype(np.float32)
    zero = (bits & 0x7FFFFFFF) == 0
    want[zero] = x[zero]
    assert_bitwise_equal(got, want, nan_equal=False)


def test_neg_flips_only_the_sign_bit():
    bits = np.array([0, 0x80000000, 0x7FC00001, 0xFF800000, 1, 0x3F800000], dtype=np.uint32)
    got = O.unary_contig(O.NEG, bits.view(np.float32)).view(np.uint32)
    assert np.array_equal(got, bits ^ 0x80000000)


def test_sum_sequential_left_fold():
    rng = _rng(9)
    x = rng.standard_normal(1000).astype(np.float32)
    want = np.float32(-0.0)
    for v in x:
        want = np.float32(want + v)
    assert O.sum_f32(x, (1000,)).view(np.uint32) == want.view(np.uint32)
    # Logical order of a transposed view, not storage order.
    y = rng.standard_normal((30, 40)).astype(np.float32)
    want = np.float32(-0.0)
    for v in y.T.ravel():
        want = np.float32(want + v)
    assert O.sum_f32(y.ravel(), (40, 30), (1, 40)).view(np.uint32) == want.view(np.uint32)


def test_reduce_to_shape_is_mul_vjp_with_ones():
    # The add VJP (new) is pinned to the reference's Multiply VJP by composition.
    rng = _rng(13)
    up = rng.standard_normal(4 * 5 * 6).astype(np.float32)
    for self_shape in [(5, 1), (1, 6), (4, 1, 6), (6,), (), (4, 5, 6)]:
        ones = np.ones(int(np.prod(self_shape)) if self_shape else 1, np.float32)
        r = O.reduce_to_shape(up, (4, 5, 6), self_shape)
        # mul VJP of operand `self` against an all-ones `other` of the output shape
        m = O.mul_backward(up, (4, 5, 6), np.ones(120, np.float32), (4, 5, 6), (30, 6, 1), 0, self_shape)
        assert_bitwise_equal(r, m)
        del ones


def test_mul_vjp_accumulation_order_is_output_major():
    # Broadcast accumulation: grad[j] = ((0 + c0) + c1) + ... over output order.
    rng = _rng(17)
    up = rng.standard_normal(3 * 4).astype(np.float32)
    other = rng.standard_normal(3 * 4).astype(np.float32)
    got = O.mul_backward(up, (3, 4), other, (3, 4), (4, 1), 0, (4,))
    want = np.zeros(4, np.float32)
    for i in range(3):
        for j in range(4):
            want[j] = np.float32(want[j] + np.float32(up[i * 4 + j] * other[i * 4 + j]))
    assert_bitwise_equal(got, want)


def test_binary_broadcast_matches_numpy_elementwise():
    # Each element is one IEEE op; numpy's float32 ops are IEEE too.
    rng = _rng(19)
    a = rng.standard_normal((4, 1, 6)).astype(np.float32)
    b = rng.standard_normal((5, 1)).astype(np.float32)
    shape, strides = O.binary_output_layout((4, 1, 6), (6, 6, 1), (5, 1), (1, 1))
    for op, fn in [(O.ADD, np.add), (O.SUB, np.subtract), (O.MUL, np.multiply), (O.DIV, np.divide)]:
        got = O.binary(op, a.ravel(), (4, 1, 6), (6, 6, 1), 0, b.ravel(), (5, 1), (1, 1), 0, shape, strides)
        assert_bitwise_equal(got, fn(a, b).ravel())


def test_libc_version_recorded():
    assert O.libc_version()


def test_row_broadcast_matches_general_broadcast_and_numpy():
    """orc_row_broadcast_f32 (the trailing-vector fast path, tensor.rs:3454-3543)
    agrees with the oracle's general odometer path and with numpy's IEEE ops."""
    rng = np.random.default_rng(21)
    rows, cols = 37, 65
    x = rng.standard_normal(rows * cols).astype(np.float32)
    v = rng.standard_normal(cols).astype(np.float32)
    for op, fn in ((O.ADD, np.add), (O.SUB, np.subtract), (O.MUL, np.multiply), (O.DIV, np.divide)):
        fast = O.row_broadcast(op, x, v, rows, cols)
        general = O.binary(op, x, (rows, cols), (cols, 1), 0, v, (cols,), (1,), 0, (rows, cols), (cols, 1))
        assert np.array_equal(fast.view(np.uint32), general.view(np.uint32))
        assert np.array_equal(fast, fn(x.reshape(rows, cols), v).ravel())


def test_mask_apply_is_two_roundings_and_keeps_signed_zeros():
    """(h * m) * s as the reference's mul then mul_scalar: two IEEE roundings,
    -x * 0 -> -0.0 (not a select), NaN * 0 -> NaN."""
    rng = np.random.default_rng(22)
    h = rng.standard_normal(4096).astype(np.float32)
    h[:4] = [-3.0, np.nan, np.inf, -0.0]
    m = (rng.random(4096) < 0.9).astype(np.uint8)
    m[:4] = 0
    s = np.float32(1 / 0.9)
    out = O.mask_apply(h, m, s)
    with np.errstate(invalid="ignore"):
        want = (h * m.astype(np.float32)) * s
    assert np.array_equal(out.view(np.uint32)[4:], want.view(np.uint32)[4:])
    assert out.view(np.uint32)[0] == 0x80000000  # -3 * 0 = -0.0
    assert out.view(np.uint32)[3] == 0x80000000  # -0 * 0 = -0.0
    assert np.isnan(out[1]) and np.isnan(out[2])  # NaN*0 and inf*0 are NaN


def test_accumulate_is_elementwise_ieee_add():
    rng = np.random.default_rng(23)
    a = rng.standard_normal(1000).astype(np.float32)
    b = rng.standard_normal(1000).astype(np.float32)
    dst = a.copy()
    O.lib().orc_accumulate_f32(dst.ctypes.data, b.ctypes.data, 1000)
    assert np.array_equal(dst, a + b)


def test_bound_helpers_are_absolute_value_products_in_double():
    rng = np.random.default_rng(24)
    a = rng.standard_normal((9, 13)).astype(np.float32)
    b = rng.standard_normal((13, 7)).astype(np.float32)
    rows = np.arange(9)
    _, bound = O.matmul_rows(a.ravel(), (9, 13), (13, 1), b.ravel(), (13, 7), (7, 1), rows)
    want = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    assert np.allclose(bound, want, rtol=1e-12, atol=0)
    assert np.isclose(O.sum_abs(a.ravel()), np.abs(a.astype(np.float64)).sum(), rtol=1e-12)


@pytest.mark.parametrize("m,k,n", [(1, 3, 5), (4, 8, 8), (7, 33, 9), (13, 64, 70)])
def test_row_blocked_matmul_is_bit_identical_to_the_plain_loop(m, k, n):
    """The 4-row blocked loop (tensor.rs:3919-3966) keeps every output's
    addition order, so it must equal the plain sequential loop bit for bit."""
    rng = _rng(40 + m)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    plain = O.matmul(a.ravel(), (m, k), (k, 1), 0, b.ravel(), (k, n), (n, 1), 0).reshape(m, n)
    blocked = O.matmul_row_blocked(a, b)
    assert_bitwise_equal(blocked, plain)


@pytest.mark.parametrize("m,k,n,threads", [(1, 3, 5, 4), (6, 17, 9, 3), (37, 64, 70, 8), (130, 41, 33, 64)])
def test_threaded_matmul_is_bit_identical_to_the_plain_loop(m, k, n, threads):
    """Splitting the row-blocked loop over threads by output rows keeps every
    element's k-ascending order, so the result equals the plain loop bit for
    bit, also with more threads than rows and rows not a multiple of 4."""
    rng = _rng(60 + m)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    plain = O.matmul(a.ravel(), (m, k), (k, 1), 0, b.ravel(), (k, n), (n, 1), 0).reshape(m, n)
    assert_bitwise_equal(O.matmul_threads(a, b, threads=threads), plain)


def _exact_exp(first_bits, n):
    x = np.arange(first_bits, first_bits + n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    return O.unary_contig(O.EXP, x)


def test_exp_checker_reports_planted_ulp_errors():
    """orc_exp_max_ulp must report the largest planted distance and where it
    is: exact glibc values give 0; values moved by known counts of
    representable floats (across thread boundaries) give those counts."""
    first = 0x3F000000  # 0.5 upward: finite, normal results
    n = 100_003
    exact = _exact_exp(first, n)
    assert O.exp_max_ulp(exact, first, threads=7) == (0, 0)
    for idx, steps in ((5, 1), (n // 2, 3), (n - 1, 2), (14_286, -4)):
        got = exact.copy()
        got.view(np.int32)[idx] += steps  # positive finite values: bits are monotone
        assert O.exp_max_ulp(got, first, threads=7) == (abs(steps), idx)
    got = exact.copy()
    got.view(np.int32)[10] += 2
    got.view(np.int32)[70_000] -= 5
    assert O.exp_max_ulp(got, first, threads=7) == (5, 70_000)


def test_exp_checker_nan_handling_and_signed_results():
    """A NaN where glibc gives a number (or the reverse) is the largest
    distance; NaN where glibc gives NaN is 0.  Distances across zero count
    the representable floats between (here at the underflow edge)."""
    first = 0x7F800000 - 8  # the last finite floats, +inf, then NaN patterns
    n = 16
    exact = _exact_exp(first, n)
    assert np.isnan(exact[-1]) and np.isinf(exact[7])
    assert O.exp_max_ulp(exact, first, threads=2)[0] == 0
    got = exact.copy()
    got[3] = np.nan
    assert O.exp_max_ulp(got, first, threads=2) == (2 ** 64 - 1, 3)
    got = exact.copy()
    got[-1] = np.float32(1.0)
    assert O.exp_max_ulp(got, first, threads=2) == (2 ** 64 - 1, n - 1)
    # exp of large negative inputs is +0.0; -0.0 counts as the same value and
    # the smallest subnormal as one float away
    first = int(np.float32(-120.0).view(np.uint32))
    exact = _exact_exp(first, 4)
    assert (exact == 0).all()
    got = exact.copy()
    got[1] = -0.0
    assert O.exp_max_ulp(got, first) == (0, 0)
    got[2] = np.float32(1e-45)
    assert O.exp_max_ulp(got, first) == (1, 2)
