"""GPU parity of trs_matmul_f32 on outputs with a short side (at most 32 rows
or columns: matrix-vector products, small-batch linear layers), which run the
streaming skinny kernel with K split over slices.

Bar (north_star), as for every matmul: exact on small integers (every partial
sum exact, so any summation order gives the integer product), and
|C_gpu - C_ref| <= 1e-5 * sqrt(K) * (|A| |B|) elementwise against the
oracle's sequential sum (src/tensor.rs:3919-3966) on normal data.
"""
import ctypes

import numpy as np
import pytest

import gpu_util as U
import oracle as O

pytestmark = pytest.mark.gpu


def _plan(ashape, astr, aoff, bshape, bstr, boff):
    from trs_backend import abi
    la, lb = abi.layout_of(ashape, astr, aoff), abi.layout_of(bshape, bstr, boff)
    oshape = tuple(ashape[:-1]) + (bshape[-1],)
    lc = abi.layout_of(oshape)
    tm, tn, tk = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    sp, bl = ctypes.c_int64(), ctypes.c_int64()
    # 256-byte-aligned stand-in addresses shifted by the offsets, as the
    # device buffers of gpu_util.matmul are.
    abi.check(abi.lib.trs_matmul_plan_f32(0x10000000000, ctypes.byref(la), 0x20000000000, ctypes.byref(lb),
                                          0x30000000000, ctypes.byref(lc), ctypes.byref(tm), ctypes.byref(tn),
                                          ctypes.byref(tk), ctypes.byref(sp), ctypes.byref(bl)))
    return tm.value, tn.value, tk.value, sp.value, bl.value


def _operands(rng, m, k, n, ta, tb, batch=0, aoff=0, boff=0, ints=True):
    nb = max(batch, 1)
    if ints:
        a = rng.integers(-3, 4, size=(nb, m, k)).astype(np.float32)
        b = rng.integers(-3, 4, size=(nb, k, n)).astype(np.float32)
    else:
        a = (rng.standard_normal((nb, m, k)) / np.sqrt(k)).astype(np.float32)
        b = rng.standard_normal((nb, k, n)).astype(np.float32)
    sa = np.concatenate([np.zeros(aoff, np.float32), (np.ascontiguousarray(a.transpose(0, 2, 1)) if ta else a).ravel()])
    sb = np.concatenate([np.zeros(boff, np.float32), (np.ascontiguousarray(b.transpose(0, 2, 1)) if tb else b).ravel()])
    ast = (1, m) if ta else (k, 1)
    bst = (1, k) if tb else (n, 1)
    if batch:
        la = ((batch, m, k), (m * k,) + ast, aoff)
        lb = ((batch, k, n), (k * n,) + bst, boff)
    else:
        la, lb = ((m, k), ast, aoff), ((k, n), bst, boff)
        a, b = a[0], b[0]
    return a, b, sa, la, sb, lb


LAYOUTS = [(False, False), (False, True), (True, False), (True, True)]


def _cu_count() -> int:
    from trs_backend import abi
    name, cus, clk = ctypes.create_string_buffer(256), ctypes.c_int(), ctypes.c_int()
    abi.check(abi.lib.trs_device_info(name, 256, ctypes.byref(cus), ctypes.byref(clk)))
    return cus.value

# (M, K, N): short side M or N from 1 to 32, K below one slice, ragged, and
# long enough to split; the long side ragged against the 64-column blocks.
SHAPES = [
    (1, 4096, 4096), (4096, 4096, 1), (8, 1000, 300), (300, 1000, 8), (16, 2048, 1000), (1000, 2048, 16),
    (17, 777, 513), (513, 777, 17), (32, 4096, 96), (96, 4096, 32), (3, 5, 7), (1, 1, 1), (31, 130, 2),
    (2, 130, 31), (1, 100003, 3), (5, 64, 4099), (24, 24, 24),
]


def test_short_sides_plan_the_skinny_kernel():
    """Rows of the short side are padded to 16 or 32 by 64 columns a block;
    33 rows go to the square tiles; K is split to fill the device.  x @ W
    with at most 8 short rows runs the VALU axpy kernel instead (below)."""
    plain = lambda m, k, n: _plan((m, k), (k, 1), 0, (k, n), (n, 1), 0)
    assert plain(9, 4096, 4096)[:2] == (16, 64) and plain(9, 4096, 4096)[3] > 1
    assert plain(4096, 100, 1)[:2] == (64, 16)
    assert plain(16, 512, 4096)[:2] == (16, 64) and plain(17, 512, 4096)[:2] == (32, 64)
    assert plain(32, 512, 4096)[:2] == (32, 64) and plain(33, 512, 4096)[:2] != (32, 64)
    assert plain(4096, 512, 32)[:2] == (64, 32)
    tm, tn, tk, s, blocks = plain(9, 4096, 4096)
    assert tk % 128 == 0 and s * tk >= 4096 and blocks == (4096 // 64) * s
    assert plain(9, 100, 4096)[3] == 1  # K shorter than one slice


@pytest.mark.parametrize("m,k,n", SHAPES)
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_skinny_small_integers_exact(m, k, n, ta, tb):
    rng = np.random.default_rng(m + 3 * k + 7 * n + 11 * ta + 13 * tb)
    a, b, sa, la, sb, lb = _operands(rng, m, k, n, ta, tb)
    got = U.matmul(sa, *la, sb, *lb)
    assert np.array_equal(got, (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))


@pytest.mark.parametrize("m,k,n", [(1, 4096, 4096), (4096, 4096, 1), (16, 3000, 700), (700, 3000, 32)])
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_skinny_normal_inputs_within_tolerance(m, k, n, ta, tb):
    rng = np.random.default_rng(91 + m + n + 2 * ta + tb)
    a, b, sa, la, sb, lb = _operands(rng, m, k, n, ta, tb, ints=False)
    got = U.matmul(sa, *la, sb, *lb)
    want = O.matmul(sa, *la, sb, *lb).reshape(m, n)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    tol = 1e-5 * np.sqrt(k) * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert (err <= tol).all(), err.max()


@pytest.mark.parametrize("aoff,boff", [(1, 0), (0, 3), (2, 2)])
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_skinny_misaligned_and_odd_strides_exact(aoff, boff, ta, tb):
    """Operands at offsets that break 16-byte alignment, and a row length of
    1,001 floats, take the scalar-load variants; still exact."""
    rng = np.random.default_rng(5 + aoff + 7 * boff + 2 * ta + tb)
    for m, k, n in [(7, 1001, 1001), (1001, 1001, 7), (1, 517, 2050)]:
        a, b, sa, la, sb, lb = _operands(rng, m, k, n, ta, tb, aoff=aoff, boff=boff)
        got = U.matmul(sa, *la, sb, *lb)
        assert np.array_equal(got, (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)), (m, k, n)


@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_skinny_batched_exact(ta, tb):
    rng = np.random.default_rng(17 + 2 * ta + tb)
    for batch, m, k, n in [(5, 4, 300, 700), (3, 700, 1500, 20), (64, 1, 512, 512), (2, 32, 8192, 64)]:
        a, b, sa, la, sb, lb = _operands(rng, m, k, n, ta, tb, batch=batch)
        got = U.matmul(sa, *la, sb, *lb)
        want = np.matmul(a.astype(np.int64), b.astype(np.int64)).astype(np.float32)
        assert np.array_equal(got.reshape(want.shape), want), (batch, m, k, n)


def test_skinny_special_values_across_slices():
    """Infinities and a NaN in different K slices of a split matrix-vector
    product and of a 20-row product: NaN and signed-infinity positions equal
    the oracle's; finite elements within tolerance.  Zero padding never meets
    a stored output, so an infinity does not spread NaN to other rows."""
    rng = np.random.default_rng(23)
    for m, k, n in [(1, 8192, 2048), (20, 8192, 300), (2048, 8192, 3)]:
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        a[0, 100] = np.inf
        a[m - 1, 6000] = -np.inf
        b[4000, n - 1] = np.nan
        b[7000, 0] = np.inf
        got = U.matmul(a.ravel(), (m, k), (k, 1), 0, b.ravel(), (k, n), (n, 1), 0)
        want = O.matmul(a.ravel(), (m, k), (k, 1), 0, b.ravel(), (k, n), (n, 1), 0).reshape(m, n)
        for pred in (np.isnan, np.isposinf, np.isneginf):
            assert np.array_equal(pred(got), pred(want)), (m, k, n, pred.__name__)
        fin = np.isfinite(want)
        with np.errstate(invalid="ignore", over="ignore"):
            bound = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
        err = np.abs(got[fin].astype(np.float64) - want[fin].astype(np.float64))
        assert (err <= 1e-5 * np.sqrt(k) * bound[fin]).all()


def test_split_products_repeated_back_to_back():
    """Split products of different shapes, each repeated three times back to
    back (their workspaces come from, and return to, the block cache in
    stream order): every call exact."""
    rng = np.random.default_rng(71)
    cases = []
    for m, k, n, ta, tb in [(1, 4096, 4096, False, False), (3, 8192, 1000, False, False), (1, 4096, 4096, False, False),
                            (2000, 6000, 5, True, False), (16, 2048, 64, False, True)]:
        a, b, sa, la, sb, lb = _operands(rng, m, k, n, ta, tb)
        want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
        assert _plan(*la, *lb)[3] > 1, (m, k, n)
        cases.append((sa, la, sb, lb, want))
    for _ in range(3):
        for sa, la, sb, lb, want in cases:
            assert np.array_equal(U.matmul(sa, *la, sb, *lb), want)


def test_dot_form_with_four_rows_or_fewer_plans_the_matrix_vector_kernel():
    """x @ W.mT (and W @ x) with at most 4 short rows, K >= 1024 and enough
    rows of W for two blocks per CU run the VALU matrix-vector kernel: the
    plan reports its 1, 2 or 4 rows by the 4 rows of W a block takes, over
    the whole of K (no split)."""
    dot = lambda m, k, n: _plan((m, k), (k, 1), 0, (k, n), (1, k), 0)
    assert dot(1, 4096, 4096)[:4] == (1, 4, 1024, 1)
    assert dot(2, 4096, 4096)[:2] == (2, 4) and dot(3, 4096, 4096)[:2] == (4, 4)
    assert dot(5, 4096, 4096)[:2] == (16, 64)       # five rows: the MFMA kernel
    assert dot(1, 512, 4096)[:2] == (16, 64)        # short K
    assert dot(1, 4096, 1024)[:2] == (16, 64)       # too few rows of W
    assert _plan((4096, 4096), (4096, 1), 0, (4096, 1), (1, 1), 0)[:2] == (4, 1)  # W @ x


def test_axpy_form_with_eight_rows_or_fewer_plans_the_valu_kernel():
    """x @ W (W unit-stride along the output columns) with at most 8 short
    rows, the long side a multiple of 4 and K >= 64 runs the VALU axpy
    kernel, compiled for 1, 2, 4 or 8 rows: the plan reports those rows by
    the 256 columns a block takes, and slices of a multiple of 64 rows for
    about one block per CU."""
    plain = lambda m, k, n: _plan((m, k), (k, 1), 0, (k, n), (n, 1), 0)
    tm, tn, tk, s, blocks = plain(1, 4096, 4096)
    assert (tm, tn) == (1, 256) and tk % 64 == 0 and s * tk >= 4096 > (s - 1) * tk and blocks == 16 * s
    assert 128 <= blocks <= 512
    assert plain(2, 4096, 4096)[:2] == (2, 256)
    assert plain(3, 4096, 4096)[:2] == (4, 256)                # three rows: the 4-row kernel
    assert plain(5, 4096, 4096)[:2] == (8, 256)
    assert plain(8, 4096, 4096)[:2] == (8, 256)
    assert plain(9, 4096, 4096)[:2] == (16, 64)               # nine rows: the MFMA kernel
    assert plain(1, 100, 4096)[:4] == (1, 256, 128, 1)        # one slice
    assert plain(1, 63, 4096)[:2] == (16, 64)                 # K < 64: the MFMA kernel
    assert plain(1, 4096, 4098)[:2] == (16, 64)               # long side not a multiple of 4
    # X strided along k (A read transposed): the VALU kernel up to 2 rows only
    at = lambda m, k, n: _plan((m, k), (1, m), 0, (k, n), (n, 1), 0)
    assert at(2, 4096, 4096)[:2] == (2, 256) and at(3, 4096, 4096)[:2] == (16, 64)
    # W^T @ x^T: the short side is N and A is read transposed (unit stride along M).
    assert _plan((4096, 4096), (1, 4096), 0, (4096, 1), (1, 1), 0)[:2] == (256, 1)


@pytest.mark.parametrize("m,k,n,ta,tb,batch", [
    (1, 4096, 4096, False, False, 0), (2, 4100, 1000, False, False, 0), (1, 777, 4100, False, False, 0),
    (2, 257, 260, False, False, 0), (1, 8192, 132, False, False, 0), (2, 64, 128, False, False, 0),
    (1, 100, 8, False, False, 0), (1, 513, 2048, False, False, 3), (2, 1000, 644, False, False, 5),
    (4096, 4096, 1, True, False, 0), (1000, 3000, 2, True, False, 0), (2048, 300, 2, True, True, 2),
    # 3..8 rows (the 4- and 8-row kernels): ragged K and long sides, batches,
    # and the W^T @ x^T form; X strided along k (A read transposed) with 2 rows
    (3, 4100, 1000, False, False, 0), (5, 777, 4100, False, False, 0), (8, 4096, 4096, False, False, 0),
    (7, 257, 260, False, False, 0), (8, 1000, 644, False, False, 5), (6, 64, 128, False, False, 0),
    (2, 1000, 300, True, False, 0), (2, 3000, 2052, True, False, 2), (4096, 4096, 8, True, True, 0),
    (1000, 3000, 5, True, True, 2),
])
def test_axpy_kernel_exact(m, k, n, ta, tb, batch):
    """The VALU axpy kernel on ragged K (slices that end early), long sides
    that leave a block's columns partly past the edge, 1 to 8 short rows,
    either side short (x @ W and W^T @ x^T), X strided along k, and batches:
    exact on small integers."""
    rng = np.random.default_rng(m + 5 * k + 11 * n + batch)
    a, b, sa, la, sb, lb = _operands(rng, m, k, n, ta, tb, batch=batch)
    assert _plan(*la, *lb)[1 if m <= n else 0] == 256, "not the axpy kernel"
    got = U.matmul(sa, *la, sb, *lb)
    want = np.matmul(a.astype(np.int64), b.astype(np.int64)).astype(np.float32)
    assert np.array_equal(got.reshape(want.shape), want)


@pytest.mark.parametrize("m,k,n,ta,tb,batch,aoff", [
    (32, 4096, 4096, False, True, 0, 0), (17, 1024, 1000, False, True, 0, 0), (24, 64, 65, False, True, 0, 1),
    (32, 4128, 4097, False, True, 2, 0), (20, 96, 130, False, True, 3, 3), (32, 32, 64, False, True, 0, 0),
    (4096, 512, 32, False, True, 0, 0), (1000, 2048, 25, False, True, 0, 2), (8, 4096, 4096, False, True, 0, 0),
    (5, 1024, 130, False, True, 2, 1), (16, 64, 65, False, True, 0, 0), (2000, 320, 12, False, True, 0, 0),
])
def test_lds_streaming_skinny_kernel_exact(m, k, n, ta, tb, batch, aoff):
    """Dot-form products with 5..32 short rows and K a multiple of 32 stream
    Y through LDS: long sides ragged against the 64-column blocks, one-slice
    and split K, batches, operands at float offsets, and the W @ x form
    (the short side N): exact on small integers."""
    rng = np.random.default_rng(m + 3 * k + 7 * n + batch + aoff)
    a, b, sa, la, sb, lb = _operands(rng, m, k, n, ta, tb, batch=batch, aoff=aoff)
    tm, tn, tk, s, blocks = _plan(*la, *lb)
    assert (min(tm, tn), max(tm, tn)) == (16 if min(m, n) <= 16 else 32, 64) and tk % 32 == 0, (tm, tn, tk)
    got = U.matmul(sa, *la, sb, *lb)
    want = np.matmul(a.astype(np.int64), b.astype(np.int64)).astype(np.float32)
    assert np.array_equal(got.reshape(want.shape), want)


def test_lds_streaming_skinny_kernel_plan_and_normal_inputs():
    """[32,4096] @ W.mT splits K into 8 slices of 512 over 64 column blocks
    (about 2 blocks per CU), and is within 1e-5 * sqrt(K) of the oracle on
    normal data."""
    if _cu_count() != 256:
        pytest.skip("the split listed is that of a 256-CU device")
    rng = np.random.default_rng(41)
    a, b, sa, la, sb, lb = _operands(rng, 32, 4096, 4096, False, True, ints=False)
    assert _plan(*la, *lb) == (32, 64, 512, 8, 512)
    got = U.matmul(sa, *la, sb, *lb)
    want = O.matmul(sa, *la, sb, *lb).reshape(32, 4096)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    tol = 1e-5 * np.sqrt(4096) * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert (err <= tol).all(), err.max()


def test_axpy_kernel_normal_inputs_within_tolerance():
    rng = np.random.default_rng(31)
    for m, k, n in [(1, 4096, 4096), (2, 4096, 4096), (2, 3000, 1000), (8, 4096, 4096), (5, 3000, 1000)]:
        a, b, sa, la, sb, lb = _operands(rng, m, k, n, False, False, ints=False)
        got = U.matmul(sa, *la, sb, *lb)
        want = O.matmul(sa, *la, sb, *lb).reshape(m, n)
        err = np.abs(got.astype(np.float64) - want.astype(np.float64))
        tol = 1e-5 * np.sqrt(k) * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
        assert (err <= tol).all(), err.max()


@pytest.mark.parametrize("m,k,n,ta,tb,aoff,boff", [
    (1, 1024, 2048, False, True, 0, 0), (2, 3000, 2050, False, True, 0, 0), (3, 4100, 2048, False, True, 0, 0),
    (4, 5000, 3001, False, True, 0, 0), (1, 70000, 2048, False, True, 0, 0),
    (2050, 3000, 2, False, False, 0, 0),   # W @ x: X = x^T with a k stride of 2 (scalar X loads)
    (3001, 1027, 4, False, True, 0, 0), (2048, 4096, 1, False, True, 0, 0),
    (1, 4096, 4096, False, True, 1, 0),    # x misaligned: float4 loads at dword alignment
    (1, 4096, 4096, False, True, 0, 1),    # W misaligned, likewise
    (1, 4097, 4096, False, True, 0, 0),    # rows of W 4097 floats apart: every other row misaligned
    (3, 4097, 4097, False, False, 0, 0),   # the axpy form's fallback (L not a multiple of 4)
])
def test_matrix_vector_kernel_exact(m, k, n, ta, tb, aoff, boff):
    rng = np.random.default_rng(m + k + n + aoff + 3 * boff)
    a, b, sa, la, sb, lb = _operands(rng, m, k, n, ta, tb, aoff=aoff, boff=boff)
    got = U.matmul(sa, *la, sb, *lb)
    assert np.array_equal(got, (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32))


@pytest.mark.parametrize("m,k,n,ta,tb", [
    (1, 4096, 4096, False, False),    # VALU axpy kernel, K split
    (1, 4096, 4096, False, True),     # VALU matrix-vector kernel
    (8, 4096, 1000, False, False),    # MFMA skinny kernel, K split, slice sum
    (32, 2048, 300, False, True),
    (64, 4096, 512, False, False),    # K split over the small tiles, float4 split sum
    (300, 1000, 500, True, False),    # edge-guarded small tiles
    (2047, 2047, 2047, False, False),  # K split, one float per lane in the slice sum
    (4096, 80, 4096, False, True),    # 256x256 tiles loaded straight into LDS, a partial last slice
    (1024, 512, 1024, True, False),   # 128x128 tiles loaded straight into LDS, K split
])
def test_result_bits_do_not_depend_on_operand_alignment(m, k, n, ta, tb):
    """Float4 loads, and the 16-byte loads straight into LDS, need only dword
    alignment, so the plan, and with it every result bit, is the same with
    the operands at any float offset."""
    got, plans = [], []
    for aoff, boff in [(0, 0), (1, 0), (0, 3), (2, 1)]:
        rng = np.random.default_rng(m * 7 + k * 3 + n)
        a, b, sa, la, sb, lb = _operands(rng, m, k, n, ta, tb, aoff=aoff, boff=boff, ints=False)
        got.append(U.matmul(sa, *la, sb, *lb))
        plans.append(_plan(*la, *lb))
    for g, p in zip(got[1:], plans[1:]):
        assert p == plans[0]
        assert np.array_equal(g.view(np.uint32), got[0].view(np.uint32))


def test_matrix_vector_kernel_batched_and_normal_inputs():
    rng = np.random.default_rng(9)
    a, b, sa, la, sb, lb = _operands(rng, 1, 2048, 2048, False, True, batch=3)
    got = U.matmul(sa, *la, sb, *lb)
    want = np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.float32)
    assert np.array_equal(got.reshape(want.shape), want)
    for m, k, n in [(1, 4096, 4096), (4, 3000, 2048)]:
        a, b, sa, la, sb, lb = _operands(rng, m, k, n, False, True, ints=False)
        got = U.matmul(sa, *la, sb, *lb)
        want = O.matmul(sa, *la, sb, *lb).reshape(m, n)
        err = np.abs(got.astype(np.float64) - want.astype(np.float64))
        tol = 1e-5 * np.sqrt(k) * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
        assert (err <= tol).all(), err.max()
