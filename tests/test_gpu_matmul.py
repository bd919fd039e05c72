"""GPU parity of trs_matmul_f32 (FP32 MFMA) against the oracle's sequential matmul.

Bar (north_star): |C_gpu - C_ref| <= 1e-5 * sqrt(K) * (|A| |B|) elementwise,
plus exact results on small integers (every partial sum exact) and the
reference's known answers (tests/tensor_baseline.rs:1212-1218, 1889-1939).
"""
import numpy as np
import pytest

import gpu_util as U
import oracle as O
from helpers import golden

pytestmark = pytest.mark.gpu
G = golden()


def _check_tol(got, want, bound, K):
    tol = 1e-5 * np.sqrt(K) * bound
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bad = err > tol
    assert not bad.any(), f"{bad.sum()} elements out of tolerance; worst {err.max()} vs {tol.ravel()[err.argmax()]}"


def _abs_bound(a, b):
    return np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)


@pytest.mark.parametrize("key", ["matmul_known", "matmul_transposed", "matmul_indexed_transposed"])
def test_known_answers(key):
    g = G[key]
    if key == "matmul_known":
        a, b = np.array(g["left"], np.float32), np.array(g["right"], np.float32)
        la = (g["left_shape"], O.contiguous_strides(g["left_shape"]), 0)
        lb = (g["right_shape"], O.contiguous_strides(g["right_shape"]), 0)
    else:
        a = np.arange(g["left_storage_len"], dtype=np.float32)
        b = np.arange(g["right_storage_len"], dtype=np.float32)
        la = (g["left_shape"], g["left_strides"], g["left_offset"])
        lb = (g["right_shape"], g["right_strides"], g["right_offset"])
    got = U.matmul(a, *la, b, *lb)
    assert got.ravel().tolist() == g["expected"]


SHAPES = [(1, 1, 1), (5, 7, 3), (64, 64, 64), (128, 128, 128), (130, 70, 257), (256, 512, 384), (33, 1000, 65)]


@pytest.mark.parametrize("m,k,n", SHAPES)
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_small_integers_exact(m, k, n, ta, tb):
    rng = np.random.default_rng(m + 3 * k + 7 * n + 11 * ta + 13 * tb)
    a = rng.integers(-4, 5, size=(m, k)).astype(np.float32)
    b = rng.integers(-4, 5, size=(k, n)).astype(np.float32)
    la = ((m, k), (1, m), 0) if ta else ((m, k), (k, 1), 0)
    lb = ((k, n), (1, k), 0) if tb else ((k, n), (n, 1), 0)
    sa = np.ascontiguousarray(a.T).ravel() if ta else a.ravel()
    sb = np.ascontiguousarray(b.T).ravel() if tb else b.ravel()
    got = U.matmul(sa, *la, sb, *lb)
    assert np.array_equal(got, (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))


@pytest.mark.parametrize("m,k,n", [(128, 256, 128), (200, 300, 100), (512, 512, 512)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True)])
def test_normal_inputs_within_tolerance(m, k, n, ta, tb):
    rng = np.random.default_rng(m * k + n)
    a = (rng.standard_normal((m, k)) / np.sqrt(k)).astype(np.float32)
    b = (rng.standard_normal((k, n)) / np.sqrt(k)).astype(np.float32)
    sa = np.ascontiguousarray(a.T).ravel() if ta else a.ravel()
    sb = np.ascontiguousarray(b.T).ravel() if tb else b.ravel()
    la = ((m, k), (1, m), 0) if ta else ((m, k), (k, 1), 0)
    lb = ((k, n), (1, k), 0) if tb else ((k, n), (n, 1), 0)
    got = U.matmul(sa, *la, sb, *lb)
    want = O.matmul(sa, *la, sb, *lb).reshape(m, n)
    _check_tol(got, want, _abs_bound(a, b), k)


def test_batched_against_per_matrix_reference():
    rng = np.random.default_rng(3)
    bt, m, k, n = 6, 96, 160, 72
    a = rng.standard_normal((bt, m, k)).astype(np.float32)
    b = rng.standard_normal((bt, k, n)).astype(np.float32)
    got = U.matmul(a.ravel(), (bt, m, k), (m * k, k, 1), 0, b.ravel(), (bt, k, n), (k * n, n, 1), 0)
    want = O.matmul(a.ravel(), (m, k), (k, 1), 0, b.ravel(), (k, n), (n, 1), 0, batch=bt, bsa=m * k, bsb=k * n)
    want = want.reshape(bt, m, n)
    for t in range(bt):
        _check_tol(got[t], want[t], _abs_bound(a[t], b[t]), k)


@pytest.mark.parametrize("m,k,n", [(20, 30, 10), (256, 512, 384), (1024, 1024, 1024)])
def test_general_strides_are_gathered_onto_the_mfma_tiles(m, k, n):
    """Operands with no unit stride are copied contiguous and multiplied on
    the MFMA tiles: exact on small integers, within the tolerance on normal
    data, and the plan reports an MFMA tile."""
    rng = np.random.default_rng(4 + m)
    la = ((m, k), (2 * k, 2), 1)   # no unit stride
    lb = ((k, n), (3 * n, 3), 2)
    ints_a = rng.integers(-3, 4, m * k * 2).astype(np.float32)
    ints_b = rng.integers(-3, 4, k * n * 3).astype(np.float32)
    got = U.matmul(ints_a, *la, ints_b, *lb)
    want = O.matmul(ints_a, *la, ints_b, *lb).reshape(m, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    buf_a = rng.standard_normal(m * k * 2).astype(np.float32)
    buf_b = rng.standard_normal(k * n * 3).astype(np.float32)
    got = U.matmul(buf_a, *la, buf_b, *lb)
    want = O.matmul(buf_a, *la, buf_b, *lb).reshape(m, n)
    a = np.lib.stride_tricks.as_strided(buf_a[1:], (m, k), (8 * k, 8))
    b = np.lib.stride_tricks.as_strided(buf_b[2:], (k, n), (12 * n, 12))
    _check_tol(got, want, _abs_bound(a, b), k)
    import ctypes
    from trs_backend import abi
    tm, tn, tk, sp, bl = (ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int64(), ctypes.c_int64())
    abi.check(abi.lib.trs_matmul_plan_f32(None, ctypes.byref(abi.layout_of(*la)), None,
                                          ctypes.byref(abi.layout_of(*lb)), None, ctypes.byref(abi.layout_of((m, n))),
                                          ctypes.byref(tm), ctypes.byref(tn), ctypes.byref(tk), ctypes.byref(sp),
                                          ctypes.byref(bl)))
    assert tm.value > 0 and tn.value > 0 and tk.value > 0


def _oracle_threads():
    import os
    return max(1, min(16, len(os.sched_getaffinity(0))))


def test_config4_full_size_every_element():
    """4096^3 with N(0, 1/64) inputs (seed 3): every element of the device
    product against the reference-order oracle (the row-blocked loop split
    over threads, bit-identical to the sequential one) within
    1e-5*sqrt(K)*(|A||B|)."""
    from trs_backend.configs import generate
    A = generate("matmul", "A")
    B = generate("matmul", "B")
    K = 4096
    got = U.matmul(A, (K, K), (K, 1), 0, B, (K, K), (K, 1), 0)
    a, b = A.reshape(K, K), B.reshape(K, K)
    want = O.matmul_threads(a, b, threads=_oracle_threads())
    _check_tol(got, want, _abs_bound(a, b), K)


def test_config4_batched_every_batch():
    """[32,512,512] @ [32,512,512] (seed 3): all 32 batches, every element."""
    from trs_backend.configs import generate
    A = generate("matmul", "Ab").reshape(32, 512, 512)
    B = generate("matmul", "Bb").reshape(32, 512, 512)
    got = U.matmul(A.ravel(), (32, 512, 512), (512 * 512, 512, 1), 0, B.ravel(), (32, 512, 512), (512 * 512, 512, 1), 0)
    for t in range(32):
        want = O.matmul_threads(A[t], B[t], threads=_oracle_threads())
        _check_tol(got[t], want, _abs_bound(A[t], B[t]), 512)


def test_inner_mismatch_and_rank_errors():
    import ctypes
    from trs_backend import abi
    a = U.dev(np.zeros(6, np.float32))
    out = U.out_buffer(4)
    rc = abi.lib.trs_matmul_f32(a.ptr, ctypes.byref(abi.layout_of((2, 3))), a.ptr, ctypes.byref(abi.layout_of((2, 3))),
                                out.ptr, ctypes.byref(abi.layout_of((2, 3))))
    assert rc == -5
    assert "mat1 and mat2 shapes cannot be multiplied (2x3 and 2x3)" in abi.lib.trs_last_error().decode()
    rc = abi.lib.trs_matmul_f32(a.ptr, ctypes.byref(abi.layout_of((6,))), a.ptr, ctypes.byref(abi.layout_of((6,))),
                                out.ptr, ctypes.byref(abi.layout_of((1,))))
    assert rc == -6


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_large_tile_all_layouts_exact_on_small_integers(ta, tb):
    """4096 x 256 @ 256 x 4096 takes the 256x256 tile path in every operand
    layout; small integers make every order of summation exact."""
    rng = np.random.default_rng(31)
    m, k, n = 4096, 256, 4096
    a = rng.integers(-3, 4, (m, k)).astype(np.float32)
    b = rng.integers(-3, 4, (k, n)).astype(np.float32)
    want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    ast, aoff = (np.ascontiguousarray(a.T), (1, m)) if ta else (a, (k, 1))
    bst, boff = (np.ascontiguousarray(b.T), (1, k)) if tb else (b, (n, 1))
    got = U.matmul(ast.ravel(), (m, k), aoff, 0, bst.ravel(), (k, n), boff, 0)
    assert np.array_equal(got, want)


def _layouts(a, b, ta, tb):
    (m, k), n = a.shape, b.shape[1]
    ast, astr = (np.ascontiguousarray(a.T), (1, m)) if ta else (a, (k, 1))
    bst, bstr = (np.ascontiguousarray(b.T), (1, k)) if tb else (b, (n, 1))
    return ast.ravel(), ((m, k), astr, 0), bst.ravel(), ((k, n), bstr, 0)


def _cu_count() -> int:
    import ctypes
    from trs_backend import abi
    name, cus, clk = ctypes.create_string_buffer(256), ctypes.c_int(), ctypes.c_int()
    abi.check(abi.lib.trs_device_info(name, 256, ctypes.byref(cus), ctypes.byref(clk)))
    return cus.value


def _plan(m, k, n, ta=False, tb=False):
    """(tile_m, tile_n, tile_k, splits, blocks) trs_matmul_f32 chooses for a
    16-byte-aligned product in the given layout on this device."""
    import ctypes
    from trs_backend import abi
    la = abi.layout_of((m, k), (1, m) if ta else (k, 1))
    lb = abi.layout_of((k, n), (1, k) if tb else (n, 1))
    lc = abi.layout_of((m, n))
    tm, tn, tk = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    sp, bl = ctypes.c_int64(), ctypes.c_int64()
    abi.check(abi.lib.trs_matmul_plan_f32(None, ctypes.byref(la), None, ctypes.byref(lb), None, ctypes.byref(lc),
                                          ctypes.byref(tm), ctypes.byref(tn), ctypes.byref(tk), ctypes.byref(sp),
                                          ctypes.byref(bl)))
    return tm.value, tn.value, tk.value, sp.value, bl.value


# Outputs with fewer 256x256 tiles than CUs and a long K.  On a 256-CU device
# K is split into S slices (the value given here) summed in slice order: S
# slices fill half the CUs, or give as many blocks as the unsplit tile.
SPLIT_K = [(256, 8192, 256, 8), (1024, 8192, 2048, 8), (4096, 8192, 1024, 4), (8192, 4096, 1024, 2)]


def _expect_split(m, k, n, s, ta, tb):
    if _cu_count() != 256:
        pytest.skip(f"the split counts listed are those of a 256-CU device (this one has {_cu_count()})")
    plan = _plan(m, k, n, ta, tb)
    assert plan[:2] == (256, 256) and plan[3] == s, plan


@pytest.mark.parametrize("m,k,n,s", SPLIT_K)
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_split_k_all_layouts_exact_on_small_integers(m, k, n, s, ta, tb):
    """The plan splits K as listed, and every partial and total sum of small
    integers is exact, so the split result equals the float64 product."""
    _expect_split(m, k, n, s, ta, tb)
    rng = np.random.default_rng(m + k + n + 2 * ta + tb)
    a = rng.integers(-3, 4, (m, k)).astype(np.float32)
    b = rng.integers(-3, 4, (k, n)).astype(np.float32)
    want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    sa, la, sb, lb = _layouts(a, b, ta, tb)
    assert np.array_equal(U.matmul(sa, *la, sb, *lb), want)


# Outputs whose 128x128 or 64x128 tile gives at most one block per CU: K is
# split over that tile for about two blocks per CU, in slices of at least 128
# k rounded up to the tile's depth (the last slice may be shorter).  The
# first three would give fewer blocks split over the 256x256 tile.  Values
# are the (tile_m, tile_n, splits) of a 256-CU device.
TILE_SPLIT = [((256, 2048, 256), (64, 128, 16)), ((1024, 4096, 1024), (64, 128, 4)),
              ((512, 4096, 1024), (64, 128, 8)), ((64, 4096, 4096), (64, 128, 16)),
              ((1000, 1000, 1000), (128, 128, 7)), ((2047, 2047, 2047), (128, 128, 2)), ((33, 1000, 65), (128, 128, 7))]


@pytest.mark.parametrize("mkn,plan", TILE_SPLIT)
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_tile_split_all_layouts_exact_on_small_integers(mkn, plan, ta, tb):
    """The plan splits as listed; slices of ragged K (1000, 2047) end short,
    and outputs of any element count (33 x 65) are summed one float per lane;
    the products are exact on small integers."""
    m, k, n = mkn
    if _cu_count() != 256:
        pytest.skip("plan expectations are those of a 256-CU device")
    got_plan = _plan(m, k, n, ta, tb)
    assert (got_plan[0], got_plan[1], got_plan[3]) == plan, got_plan
    rng = np.random.default_rng(m + n + 2 * ta + tb)
    a = rng.integers(-3, 4, (m, k)).astype(np.float32)
    b = rng.integers(-3, 4, (k, n)).astype(np.float32)
    want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    sa, la, sb, lb = _layouts(a, b, ta, tb)
    assert np.array_equal(U.matmul(sa, *la, sb, *lb), want)


@pytest.mark.parametrize("m,k,n", [(1000, 1000, 1000), (64, 4096, 4096)])
def test_tile_split_normal_inputs_within_tolerance(m, k, n):
    rng = np.random.default_rng(31 + m)
    a = (rng.standard_normal((m, k)) / np.sqrt(k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    got = U.matmul(a.ravel(), (m, k), (k, 1), 0, b.ravel(), (k, n), (n, 1), 0)
    want = O.matmul_threads(a, b, threads=_oracle_threads())
    _check_tol(got, want, _abs_bound(a, b), k)


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_split_k_normal_inputs_within_tolerance(ta, tb):
    m, k, n = 256, 8192, 256
    _expect_split(m, k, n, 8, ta, tb)
    rng = np.random.default_rng(77 + 2 * ta + tb)
    a = (rng.standard_normal((m, k)) / np.sqrt(k)).astype(np.float32)
    b = (rng.standard_normal((k, n)) / np.sqrt(k)).astype(np.float32)
    sa, la, sb, lb = _layouts(a, b, ta, tb)
    got = U.matmul(sa, *la, sb, *lb)
    # The reference's order does not depend on the operands' layout: the
    # oracle runs on the logical matrices.
    want = O.matmul_threads(a, b, threads=_oracle_threads())
    _check_tol(got, want, _abs_bound(a, b), k)


def test_split_k_special_values_across_slices():
    """Infinities and a NaN in different k slices: NaN and signed-infinity
    positions equal the oracle's sequential sum; the rest within tolerance."""
    m, k, n = 256, 8192, 256
    _expect_split(m, k, n, 8, False, False)
    rng = np.random.default_rng(5)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    a[5, 100], a[5, 6000], a[7, 4000], a[9, 2100] = np.inf, -np.inf, np.nan, np.inf
    b[3500, 9] = -np.inf
    got = U.matmul(a.ravel(), (m, k), (k, 1), 0, b.ravel(), (k, n), (n, 1), 0)
    want = O.matmul(a.ravel(), (m, k), (k, 1), 0, b.ravel(), (k, n), (n, 1), 0).reshape(m, n)
    for pred in (np.isnan, np.isposinf, np.isneginf):
        assert np.array_equal(pred(got), pred(want))
    assert np.isnan(want[5]).any() and np.isnan(want[7]).all() and np.isinf(want[:, 9]).sum() > 200
    fin = np.isfinite(want)
    with np.errstate(invalid="ignore", over="ignore"):
        bound = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    err = np.abs(got[fin].astype(np.float64) - want[fin].astype(np.float64))
    assert (err <= 1e-5 * np.sqrt(k) * bound[fin]).all()


def test_random_shapes_layouts_and_offsets_exact_on_small_integers():
    """40 random products: M, N, K in 1-300 (ragged edge tiles), each operand
    plain or transposed (.mT) and at a random storage offset, rank 2 or a
    batch of 1-3.  Small-integer entries make every partial sum exact, so the
    GPU result equals the integer product bit for bit."""
    rng = np.random.default_rng(808)
    for case in range(40):
        m, k, n = (int(rng.integers(1, 301)) for _ in range(3))
        batch = int(rng.integers(1, 4)) if rng.random() < 0.4 else 0
        ta, tb = bool(rng.random() < 0.5), bool(rng.random() < 0.5)
        oa, ob = int(rng.integers(0, 5)), int(rng.integers(0, 5))
        nb = max(batch, 1)
        a = rng.integers(-3, 4, size=(nb, m, k)).astype(np.float32)
        b = rng.integers(-3, 4, size=(nb, k, n)).astype(np.float32)
        sa = np.concatenate([np.zeros(oa, np.float32), (np.ascontiguousarray(a.transpose(0, 2, 1)) if ta else a).ravel()])
        sb = np.concatenate([np.zeros(ob, np.float32), (np.ascontiguousarray(b.transpose(0, 2, 1)) if tb else b).ravel()])
        ast = (1, m) if ta else (k, 1)
        bst = (1, k) if tb else (n, 1)
        if batch:
            la = ((batch, m, k), (m * k,) + ast, oa)
            lb = ((batch, k, n), (k * n,) + bst, ob)
        else:
            la, lb = ((m, k), ast, oa), ((k, n), bst, ob)
        got = U.matmul(sa, *la, sb, *lb).reshape(-1)
        want = np.matmul(a.astype(np.int64), b.astype(np.int64)).astype(np.float32).reshape(-1)
        assert np.array_equal(got, want), (case, m, k, n, batch, ta, tb, oa, ob)


def test_special_values_propagate_as_the_reference():
    """src/tensor.rs:4711-4815 vectors on the GPU: NaN and signed-infinity
    positions equal the oracle's exactly; finite elements are within the
    matmul tolerance.  Element 0 of the first product (1e20 - 1e20 + 1) may
    legitimately differ from the sequential 1.0, by cancellation in MFMA
    order, within the bound 1e-5*sqrt(K)*(|A||B|)."""
    from helpers import f32_from_bits
    g = G["matmul_contiguous_specials"]
    cases = [(f32_from_bits(g["left_bits"]).reshape(2, 3), f32_from_bits(g["right_bits"]).reshape(3, 3))]
    g = G["matmul_blocked_pattern"]
    rows, inner, cols, fb = g["rows"], g["inner"], g["columns"], g["finite_bits"]
    left = f32_from_bits([fb[(i * 5 + i // inner) % 8] for i in range(rows * inner)]).reshape(rows, inner)
    special = {(3, 7): 0x7F800000, (4, 11): 0xFF800000, (5, 13): 0x7FC12345}
    right = f32_from_bits([special.get((c % 8, d), fb[(d * 3 + c) % 8]) for d in range(inner) for c in range(cols)])
    cases.append((left, right.reshape(inner, cols)))
    for a, b in cases:
        m, k = a.shape
        n = b.shape[1]
        got = U.matmul(a.ravel(), (m, k), (k, 1), 0, b.ravel(), (k, n), (n, 1), 0).reshape(m, n)
        want = O.matmul(a.ravel(), (m, k), (k, 1), 0, b.ravel(), (k, n), (n, 1), 0).reshape(m, n)
        assert np.array_equal(np.isnan(got), np.isnan(want))
        assert np.array_equal(np.isposinf(got), np.isposinf(want))
        assert np.array_equal(np.isneginf(got), np.isneginf(want))
        fin = np.isfinite(want)
        with np.errstate(invalid="ignore", over="ignore"):
            bound = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
        tol = 1e-5 * np.sqrt(k) * bound
        assert (np.abs(got[fin].astype(np.float64) - want[fin].astype(np.float64)) <= tol[fin]).all()


def test_empty_dimensions_on_the_device():
    """src/tensor.rs:4817-4839 through torch_rs on the GPU: empty outputs
    keep their shapes; K = 0 gives +0.0 everywhere (no launch reads A or B)."""
    import torch_rs
    no_rows = torch_rs.zeros((0, 3), device="cuda") @ torch_rs.ones((3, 4), device="cuda")
    assert no_rows.shape == (0, 4) and no_rows.numel() == 0
    no_cols = torch_rs.ones((2, 3), device="cuda") @ torch_rs.zeros((3, 0), device="cuda")
    assert no_cols.shape == (2, 0) and no_cols.numel() == 0
    no_inner = torch_rs.ones((2, 0), device="cuda") @ torch_rs.zeros((0, 4), device="cuda")
    assert no_inner.shape == (2, 4)
    assert (no_inner.numpy().view(np.uint32) == 0).all()


# Ragged products on the 256x256 tile (edge tiles moved back inside the
# matrix, slices loaded straight into LDS from rows of any length), and
# single matrices that exceed a multiple of 256 by at most 32 rows or columns,
# whose rims run as skinny products.  Plans are those of a 256-CU device.
RAGGED_LARGE = [
    ((4095, 300, 4095), 0, (256, 256, 16, 1, 256)),     # 255-wide rim tiles, K tail of 12
    ((1000, 50, 1000), 16, (256, 256, 16, 1, 256)),     # a batch of ragged outputs
    ((4096, 4097, 4096), 0, (256, 256, 16, 1, 256)),    # ragged K only: one 1-deep tail slice
    ((4097, 300, 4097), 0, (256, 256, 16, 1, 256)),     # one-row and one-column rims
    ((4096 + 31, 129, 4096), 0, (256, 256, 16, 1, 256)),   # a 31-row rim, full-width tile
    ((4096, 77, 4096 + 5), 0, (256, 256, 16, 1, 256)),     # a 5-column rim
    ((4352 + 3, 65, 4096 + 32), 0, (256, 256, 16, 1, 272)),  # both rims, 17 x 16 main tiles
    ((4094, 100, 4093), 0, (256, 256, 16, 1, 256)),     # edge tiles 254 x 253: straddling chunks
    ((3841, 64, 3842), 0, (256, 256, 16, 1, 256)),      # edge tiles of 1 row and 2 columns, moved back 255 and 254
]


@pytest.mark.parametrize("mkn,batch,plan", RAGGED_LARGE)
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_ragged_large_tile_and_rims_exact_on_small_integers(mkn, batch, plan, ta, tb):
    m, k, n = mkn
    if _cu_count() != 256:
        pytest.skip("plan expectations are those of a 256-CU device")
    rng = np.random.default_rng(m + 3 * k + 7 * n + batch + 2 * ta + tb)
    nb = max(batch, 1)
    a = rng.integers(-3, 4, (nb, m, k)).astype(np.float32)
    b = rng.integers(-3, 4, (nb, k, n)).astype(np.float32)
    sa = (np.ascontiguousarray(a.transpose(0, 2, 1)) if ta else a).ravel()
    sb = (np.ascontiguousarray(b.transpose(0, 2, 1)) if tb else b).ravel()
    ast, bst = ((1, m) if ta else (k, 1)), ((1, k) if tb else (n, 1))
    if batch:
        la, lb = ((batch, m, k), (m * k,) + ast, 0), ((batch, k, n), (k * n,) + bst, 0)
    else:
        la, lb = ((m, k), ast, 0), ((k, n), bst, 0)
        assert _plan(m, k, n, ta, tb) == plan
    got = U.matmul(sa, *la, sb, *lb).reshape(nb, m, n)
    want = np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.float32)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("m,k,n,batch", [(1001, 300, 1003, 16), (1002, 77, 1000, 16), (4094, 100, 4093, 0)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_ragged_large_tile_bits_match_the_padded_product(m, k, n, batch, ta, tb):
    """The 256x256 tile on ragged M and N (the last tile row and column moved
    back to end at the matrix's edge, each storing only the outputs past the
    tile before it) gives every element the bits it has in the product of
    the operands zero-padded to whole tiles: the same k steps.  Edge tiles of
    233, 234 and 254 rows and 235, 232 and 253 columns (every residue mod 4,
    so every float offset of the moved tiles' rows), in all four layouts,
    with normal inputs and a partial last slice."""
    if _cu_count() != 256:
        pytest.skip("the ragged shapes take the 256x256 tile on a 256-CU device")
    rng = np.random.default_rng(m + 5 * k + 11 * n + 2 * ta + tb)
    nb = max(batch, 1)
    mp, np_ = -(-m // 256) * 256, -(-n // 256) * 256
    a = np.zeros((nb, mp, k), np.float32)
    b = np.zeros((nb, k, np_), np.float32)
    a[:, :m] = rng.standard_normal((nb, m, k)).astype(np.float32)
    b[:, :, :n] = rng.standard_normal((nb, k, n)).astype(np.float32)

    def run(mm, nn):
        aa, bb = np.ascontiguousarray(a[:, :mm]), np.ascontiguousarray(b[:, :, :nn])
        sa = (np.ascontiguousarray(aa.transpose(0, 2, 1)) if ta else aa).ravel()
        sb = (np.ascontiguousarray(bb.transpose(0, 2, 1)) if tb else bb).ravel()
        ast, bst = ((1, mm) if ta else (k, 1)), ((1, k) if tb else (nn, 1))
        if batch:
            la, lb = ((batch, mm, k), (mm * k,) + ast, 0), ((batch, k, nn), (k * nn,) + bst, 0)
        else:
            la, lb = ((mm, k), ast, 0), ((k, nn), bst, 0)
            assert _plan(mm, k, nn, ta, tb) == (256, 256, 16, 1, 256)
        return U.matmul(sa, *la, sb, *lb).reshape(nb, mm, nn)

    got, padded = run(m, n), run(mp, np_)
    assert np.array_equal(got.view(np.uint32), padded[:, :m, :n].view(np.uint32))


# Stream-K on the 256x256 tile: one block per CU takes an equal share of the
# product's (tile, k-slice) units, and a second pass adds, in k order, the
# pieces of the tiles split between blocks.  Plans of a 256-CU device
# (splits 0 = stream-K, 256 blocks).
STREAM_K = [
    ((3072, 1024, 3072), 0, 16),   # 144 tiles for 256 CUs: two or three pieces per tile
    ((512, 4096, 4096), 0, 32),    # 32 tiles, eight pieces each
    ((2999, 1000, 2901), 0, 16),   # edge tiles 183 x 85 (straddling chunks), a K tail of 8
    ((1000, 2048, 1000), 6, 16),   # a batch of ragged outputs, 96 tiles
]


@pytest.mark.parametrize("mkn,batch,bk", STREAM_K)
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_stream_k_exact_on_small_integers(mkn, batch, bk, ta, tb):
    m, k, n = mkn
    if _cu_count() != 256:
        pytest.skip("plan expectations are those of a 256-CU device")
    rng = np.random.default_rng(m + 3 * k + 7 * n + batch + 2 * ta + tb)
    nb = max(batch, 1)
    a = rng.integers(-3, 4, (nb, m, k)).astype(np.float32)
    b = rng.integers(-3, 4, (nb, k, n)).astype(np.float32)
    sa = (np.ascontiguousarray(a.transpose(0, 2, 1)) if ta else a).ravel()
    sb = (np.ascontiguousarray(b.transpose(0, 2, 1)) if tb else b).ravel()
    ast, bst = ((1, m) if ta else (k, 1)), ((1, k) if tb else (n, 1))
    if batch:
        la, lb = ((batch, m, k), (m * k,) + ast, 0), ((batch, k, n), (k * n,) + bst, 0)
    else:
        la, lb = ((m, k), ast, 0), ((k, n), bst, 0)
        # depth 32 only with A not transposed
        assert _plan(m, k, n, ta, tb) == (256, 256, 16 if ta else bk, 0, 256)
    got = U.matmul(sa, *la, sb, *lb).reshape(nb, m, n)
    want = np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.float32)
    assert np.array_equal(got, want)


def test_stream_k_normal_inputs_within_tolerance_and_deterministic():
    """A ragged stream-K product with N(0, 1/sqrt(K)) entries: every element
    against the reference-order oracle within 1e-5*sqrt(K)*(|A||B|), and the
    same bits from a second call."""
    m, k, n = 2999, 1000, 2901
    rng = np.random.default_rng(77)
    a = (rng.standard_normal((m, k)) / np.sqrt(k)).astype(np.float32)
    b = (rng.standard_normal((k, n)) / np.sqrt(k)).astype(np.float32)
    got = U.matmul(a.ravel(), (m, k), (k, 1), 0, b.ravel(), (k, n), (n, 1), 0)
    again = U.matmul(a.ravel(), (m, k), (k, 1), 0, b.ravel(), (k, n), (n, 1), 0)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    want = O.matmul_threads(a, b, threads=_oracle_threads())
    _check_tol(got.reshape(m, n), want.reshape(m, n), _abs_bound(a, b), k)


@pytest.mark.parametrize("s", [4095, 4097])
def test_ragged_cubes_normal_inputs_within_tolerance(s):
    """4095^3 (edge tiles) and 4097^3 (a 4096^3 tile product and two rims)
    with N(0, 1/sqrt(K)) entries: every element against the reference-order
    oracle within 1e-5*sqrt(K)*(|A||B|)."""
    rng = np.random.default_rng(s)
    a = (rng.standard_normal((s, s)) / np.sqrt(s)).astype(np.float32)
    b = (rng.standard_normal((s, s)) / np.sqrt(s)).astype(np.float32)
    got = U.matmul(a.ravel(), (s, s), (s, 1), 0, b.ravel(), (s, s), (s, 1), 0)
    want = O.matmul_threads(a, b, threads=_oracle_threads())
    _check_tol(got, want, _abs_bound(a, b), s)


def _matmul_without_allocations(a, ashape, astr, aoff, b, bshape, bstr, boff):
    """U.matmul with trs_alloc refusing every request while the product runs
    (the operands and output are allocated before the hook is set)."""
    import ctypes
    from trs_backend import abi
    da, db = U.dev(a), U.dev(b)
    oshape = tuple(ashape[:-1]) + (bshape[-1],)
    n = int(np.prod(oshape))
    do = U.out_buffer(n)
    abi.check(abi.lib.trs_debug_fail_allocs_after(0))
    try:
        abi.check(abi.lib.trs_matmul_f32(da.ptr, ctypes.byref(abi.layout_of(ashape, astr, aoff)), db.ptr,
                                         ctypes.byref(abi.layout_of(bshape, bstr, boff)), do.ptr,
                                         ctypes.byref(abi.layout_of(oshape))))
    finally:
        abi.check(abi.lib.trs_debug_fail_allocs_after(-1))
    return do.to_numpy(count=n).reshape(oshape)


def test_fallbacks_when_no_workspace_can_be_allocated():
    """With every allocation refused (trs_debug_fail_allocs_after(0)):
    operands with no unit stride run the one-lane-per-output kernel, which
    adds k in the reference's order from +0.0, so it equals the oracle bit
    for bit on normal data; products whose plan splits K (over the large
    tile, the small tile, a skinny kernel, and the rims of a peeled product)
    run unsplit, exact on small integers."""
    import ctypes
    from trs_backend import abi
    rng = np.random.default_rng(2024)
    # a[::2, ::2] and b[::3, ::2]: no unit stride in either operand.
    m, k, n = 70, 90, 50
    ab = rng.standard_normal((2 * m, 2 * k)).astype(np.float32)
    bb = rng.standard_normal((3 * k, 2 * n)).astype(np.float32)
    la, lb = ((m, k), (4 * k, 2), 0), ((k, n), (6 * n, 2), 0)
    got = _matmul_without_allocations(ab.ravel(), *la, bb.ravel(), *lb)
    want = O.matmul(ab.ravel(), *la, bb.ravel(), *lb).reshape(m, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    cases = [(1024, 8192, 1024, False, False), (1000, 1000, 1000, False, False), (1, 4096, 4096, False, False),
             (32, 4096, 4096, False, True), (4097, 300, 4097, False, False), (2999, 1000, 2901, False, False)]
    for m, k, n, ta, tb in cases:
        assert _plan(m, k, n, ta, tb)[3] != 1 or m == 4097, (m, k, n)
        a = rng.integers(-3, 4, (m, k)).astype(np.float32)
        b = rng.integers(-3, 4, (k, n)).astype(np.float32)
        sa, la, sb, lb = _layouts(a, b, ta, tb)
        got = _matmul_without_allocations(sa, *la, sb, *lb)
        assert np.array_equal(got, (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)), (m, k, n)
    # the hook is off again: an allocation succeeds
    p = ctypes.c_void_p()
    abi.check(abi.lib.trs_alloc(64, ctypes.byref(p)))
    abi.check(abi.lib.trs_free(p))
