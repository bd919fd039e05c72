"""Concurrency and large-size robustness of the C ABI on the GPU.

ctypes releases the GIL for foreign calls, so the threads below really do
call into libtrs_hip.so at the same time; every call's work still lands in
order on the device stream and must give the same results as a lone call.
The large-size case drives the flat kernels past 2^32 elements (64-bit
offsets and the grid-stride continuation beyond the one-shot grid).
"""
import ctypes
import threading

import numpy as np
import pytest

import gpu_util as U
from helpers import assert_bitwise_equal
import oracle as O
from trs_backend import abi
from trs_backend.abi import DeviceArray, check, layout_of

pytestmark = pytest.mark.gpu


def test_concurrent_sums_and_ops_from_threads_match_serial_results():
    rng = np.random.default_rng(41)
    arrays = [rng.standard_normal(1 << 20).astype(np.float32) * (i + 1) for i in range(8)]
    devs = [DeviceArray.from_numpy(a) for a in arrays]
    lay = layout_of((1 << 20,))
    outs = [DeviceArray(4) for _ in arrays]

    def serial(i):
        check(abi.lib.trs_sum_f32(devs[i].ptr, ctypes.byref(lay), outs[i].ptr))
        return outs[i].to_numpy(count=1)[0]

    want = [serial(i) for i in range(8)]
    errors, got = [], {}
    barrier = threading.Barrier(8)

    def worker(i):
        try:
            barrier.wait()
            res = []
            scratch = DeviceArray((1 << 20) * 4)
            for _ in range(50):
                # interleave a pointwise op with the two-pass sum
                check(abi.lib.trs_unary_f32(3, devs[i].ptr, ctypes.byref(lay), scratch.ptr, ctypes.byref(lay)))
                check(abi.lib.trs_sum_f32(scratch.ptr, ctypes.byref(lay), outs[i].ptr))
                res.append(outs[i].to_numpy(count=1)[0])
            got[i] = res
        except Exception as e:  # reported below
            errors.append(repr(e))

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors
    for i in range(8):
        assert all(np.float32(v).view(np.uint32) == np.float32(want[i]).view(np.uint32) for v in got[i]), i


def test_flat_kernels_beyond_two_to_the_32_elements():
    n = (1 << 32) + 7
    period = 65521
    step = 1 << 28
    base = (np.arange(step + period, dtype=np.int64) % period).astype(np.float32)  # x[i] = i mod 65521
    x = np.empty(n, dtype=np.float32)
    for s in range(0, n, step):
        e = min(n, s + step)
        x[s:e] = base[s % period: s % period + (e - s)]
    dx = DeviceArray.from_numpy(x)
    del x
    dout = DeviceArray(n * 4)
    lay = layout_of((n,))
    check(abi.lib.trs_binary_scalar_f32(2, dx.ptr, ctypes.byref(lay), ctypes.c_float(0.5), dout.ptr,
                                        ctypes.byref(lay)))
    del dx
    out = dout.to_numpy(count=n)
    half = O.scalar_contig(O.S_MUL, base, 0.5)  # the oracle's (i mod 65521) * 0.5
    for s in range(0, n, step):
        e = min(n, s + step)
        assert np.array_equal(out[s:e], half[s % period: s % period + (e - s)]), s
    del dout
    check(abi.lib.trs_empty_cache())  # hand the 32 GiB back to HIP for the tests that follow


def _put(big, off, arr):
    """Copy `arr` into the allocation `big` at element offset `off`."""
    arr = np.ascontiguousarray(arr, dtype=np.float32)
    check(abi.lib.trs_memcpy_h2d(ctypes.c_void_p(big.addr + off * 4), arr.ctypes.data, arr.nbytes))


def _get(big, off, n):
    out = np.empty(n, dtype=np.float32)
    check(abi.lib.trs_memcpy_d2h(out.ctypes.data, ctypes.c_void_p(big.addr + off * 4), n * 4))
    return out


def test_row_and_transposing_layouts_on_both_sides_of_two_to_the_32_element_offsets():
    """Rank-2, rank-3 and rank-4 row launches and the rank-3 transposing one
    are compiled with 32-bit offsets when every element offset of the launch is
    below 2^32, else they take the run-time path with 64-bit offsets.  Each
    layout runs with its views ending exactly at element 2^32 - 1 of one
    allocation (32-bit) and again past 2^32 (64-bit), bit-exact against the
    oracle on the same values."""
    two32 = 1 << 32
    big = DeviceArray((two32 + (1 << 22)) * 4)
    rng = np.random.default_rng(77)
    # (name, op, left (shape, strides), right (shape, strides), output shape):
    # the left operand and the output live in `big`, the right one apart.
    cases = [
        ("rows rank 2", O.ADD, ((300, 2112), None), ((2112,), None), (300, 2112)),
        ("rows rank 3", O.MUL, ((8, 1, 1024), None), ((96, 1024), None), (8, 96, 1024)),
        ("rows rank 4", O.ADD, ((4, 1, 8, 1024), None), ((6, 1, 1024), None), (4, 6, 8, 1024)),
        ("transposed rank 3", O.SUB, ((8, 192, 320), (320 * 192, 1, 192)), ((8, 192, 320), None), (8, 192, 320)),
    ]
    for name, op, (lsh, lst), (rsh, rst), osh in cases:
        lst = lst or O.contiguous_strides(lsh)
        rst = rst or O.contiguous_strides(rsh)
        ln = O.storage_size(lsh, lst)
        on = int(np.prod(osh))
        l = rng.standard_normal(ln).astype(np.float32)
        r = rng.standard_normal(O.storage_size(rsh, rst)).astype(np.float32)
        ostr = O.contiguous_strides(osh)
        want = O.binary(op, l, lsh, lst, 0, r, rsh, rst, 0, osh, ostr)
        dr = DeviceArray.from_numpy(r)
        # output ending at element 2^32 - 1, left operand just below it; then
        # both past 2^32
        for loff, ooff in [(two32 - on - ln - 64, two32 - on), (two32 + 64, two32 + ln + 128)]:
            _put(big, loff, l)
            check(abi.lib.trs_binary_f32(op, big.ptr, ctypes.byref(layout_of(lsh, lst, loff)), dr.ptr,
                                         ctypes.byref(layout_of(rsh, rst)), big.ptr,
                                         ctypes.byref(layout_of(osh, ostr, ooff))))
            got = _get(big, ooff, on)
            assert np.array_equal(got.view(np.uint32), want.reshape(-1).view(np.uint32)), (name, ooff)
        del dr
    del big
    check(abi.lib.trs_empty_cache())


def test_outputs_may_alias_inputs_only_as_the_same_view():
    """In place is allowed element for element; any other overlap with an
    input (shifted, transposed, broadcast) or with a matmul operand is
    rejected on the host before anything is launched."""
    rng = np.random.default_rng(9)
    a = rng.standard_normal(64 * 64).astype(np.float32)
    b = rng.standard_normal(64 * 64).astype(np.float32)
    da, db = DeviceArray.from_numpy(a), DeviceArray.from_numpy(b)
    sq = layout_of((64, 64))
    # a = a + b in place: the same view
    check(abi.lib.trs_binary_f32(0, da.ptr, ctypes.byref(sq), db.ptr, ctypes.byref(sq), da.ptr, ctypes.byref(sq)))
    assert np.array_equal(da.to_numpy(), a + b)
    # accumulate is in place by construction
    check(abi.lib.trs_accumulate_f32(da.ptr, db.ptr, a.size))
    assert np.array_equal(da.to_numpy(), (a + b) + b)
    shifted = layout_of((64, 63), (64, 1), 1)
    first = layout_of((64, 63))
    rc = abi.lib.trs_binary_f32(0, da.ptr, ctypes.byref(first), db.ptr, ctypes.byref(first), da.ptr,
                                ctypes.byref(shifted))
    assert rc == abi.TRS_E_INVALID_ARGUMENT and b"overlaps input 0" in abi.lib.trs_last_error()
    transposed = layout_of((64, 64), (1, 64))
    rc = abi.lib.trs_unary_f32(3, da.ptr, ctypes.byref(transposed), da.ptr, ctypes.byref(sq))
    assert rc == abi.TRS_E_INVALID_ARGUMENT
    row = layout_of((64,))
    rc = abi.lib.trs_binary_f32(0, db.ptr, ctypes.byref(sq), da.ptr, ctypes.byref(row), da.ptr, ctypes.byref(sq))
    assert rc == abi.TRS_E_INVALID_ARGUMENT  # a broadcast row of the output's own memory
    rc = abi.lib.trs_matmul_f32(da.ptr, ctypes.byref(sq), db.ptr, ctypes.byref(sq), da.ptr, ctypes.byref(sq))
    assert rc == abi.TRS_E_INVALID_ARGUMENT and b"overlaps an operand" in abi.lib.trs_last_error()
    # the rejected calls changed nothing
    assert np.array_equal(da.to_numpy(), (a + b) + b)


def test_layouts_whose_offsets_overflow_are_rejected_before_launch():
    """IndexCalculationOverflow (src/tensor.rs:3815-3841): a view whose last
    offset, byte offset or element count leaves 64 bits is refused; a
    zero-element view addresses nothing and is accepted."""
    d = DeviceArray(4096)
    huge_stride = layout_of((4,), (1 << 62,))
    rc = abi.lib.trs_unary_f32(1, d.ptr, ctypes.byref(huge_stride), d.ptr, ctypes.byref(layout_of((4,))))
    assert rc == -2 and b"overflow" in abi.lib.trs_last_error()
    byte_overflow = layout_of((2,), (1 << 61,))
    out = DeviceArray(64)
    rc = abi.lib.trs_unary_f32(1, d.ptr, ctypes.byref(byte_overflow), out.ptr, ctypes.byref(layout_of((2,))))
    assert rc == -2
    many = layout_of((1 << 32, 1 << 32), (0, 0))
    rc = abi.lib.trs_sum_f32(d.ptr, ctypes.byref(many), out.ptr)
    assert rc == -2 and b"element count" in abi.lib.trs_last_error()
    empty = layout_of((0, (1 << 62), 3), ((1 << 62), 3, 1))
    check(abi.lib.trs_unary_f32(1, d.ptr, ctypes.byref(empty), out.ptr, ctypes.byref(empty)))


def test_allocation_failure_is_reported_and_the_library_keeps_working():
    """AllocationFailed (src/tensor.rs:5540-5580 forces it with elements =
    usize::MAX): an impossible request fails with the allocation code, after
    the block cache has been released and the allocation retried, and later
    work is unaffected."""
    import torch_rs
    p = ctypes.c_void_p()
    rc = abi.lib.trs_alloc(1 << 52, ctypes.byref(p))
    assert rc == -1 and not p.value
    assert abi.lib.trs_last_error()
    with pytest.raises(RuntimeError):
        torch_rs.zeros((1 << 40,), device="cuda")
    x = torch_rs.tensor(np.arange(8, dtype=np.float32), device="cuda")
    assert (x * 2.0).numpy().tolist() == [float(2 * i) for i in range(8)]


def test_square_sum_backward_smoke_matches_closed_form_and_is_fast():
    """The reference's only timing test (tests/test_autograd.py:1843-1867):
    (v*v).sum().backward() on 16,384 values, median of 7 timed runs after 3
    warm-ups, with a checksum of the gradients.  Here the gradient 2v is exact,
    so the checksum sum((2v)^2) is checked against float64, and the median is
    held to 2 ms (a device step measures about 30 us)."""
    import statistics
    import time
    import torch_rs
    values = np.linspace(-2.0, 2.0, 16_384, dtype=np.float32)
    inputs = [torch_rs.tensor(values, device="cuda", requires_grad=True) for _ in range(10)]
    samples, checksum = [], 0.0
    for i, v in enumerate(inputs):
        t0 = time.perf_counter()
        (v * v).sum().backward()
        torch_rs.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        g = v.grad.numpy().astype(np.float64)
        assert np.array_equal(g, 2.0 * values.astype(np.float64))
        checksum += float((g * g).sum())
        if i >= 3:
            samples.append(elapsed)
    want = 10 * float(((2.0 * values.astype(np.float64)) ** 2).sum())
    assert abs(checksum - want) <= 1e-9 * want
    assert statistics.median(samples) < 2e-3


def test_grid_stride_loops_of_every_pointwise_kernel_bit_exact():
    """Launches capped at a few blocks (trs_debug_pointwise_grid_cap), so each
    block loops over many tiles: the flat kernels (contiguous, broadcast,
    scalar tail), the rows kernel (vector on one-wave and wider blocks,
    scalar), the transposing kernel (eager, and fused with a held operand
    walked over outer tuples) and the generic kernel, each bit-exact against
    the oracle.  Without the cap only launches of more than 2^22 blocks loop."""
    rng = np.random.default_rng(77)

    def bin_case(ash, ast, aoff, bsh, bst, boff, op=O.ADD):
        a = U.special_mix(rng, O.storage_size(ash, ast, aoff))
        b = U.special_mix(rng, O.storage_size(bsh, bst, boff))
        osh, ost = O.binary_output_layout(ash, ast, bsh, bst)
        want = O.binary(op, a, ash, ast, aoff, b, bsh, bst, boff, osh, ost)
        return (op, a, ash, ast, aoff, b, bsh, bst, boff, osh, ost), want

    cs = O.contiguous_strides
    cases = {
        "flat_contig_tail": bin_case((100_003,), (1,), 0, (100_003,), (1,), 0),
        "flat_broadcast": bin_case((50_000,), (1,), 0, (), (), 0, O.MUL),
        "rows_one_wave": bin_case((300, 1028), cs((300, 1028)), 0, (1028,), (1,), 0),
        "rows_wider_blocks": bin_case((6, 1, 516), cs((6, 1, 516)), 0, (1, 40, 516), cs((1, 40, 516)), 0),
        "rows_scalar": bin_case((333, 37), cs((333, 37)), 0, (37,), (1,), 0),
        "xpose": bin_case((300, 260), (1, 300), 0, (300, 260), cs((300, 260)), 0),
        "generic": bin_case((5000,), (3,), 1, (5000,), (2,), 0),
    }
    B, M, N = 16, 96, 160
    a = rng.standard_normal(B * N).astype(np.float32)
    b = rng.standard_normal(M * N).astype(np.float32)
    c = rng.standard_normal(B * N * M).astype(np.float32)
    sh1, st1 = O.binary_output_layout((B, 1, N), (N, N, 1), (1, M, N), (M * N, N, 1))
    s1 = O.binary(O.ADD, a, (B, 1, N), (N, N, 1), 0, b, (1, M, N), (M * N, N, 1), 0, sh1, st1)
    sh2, st2 = O.binary_output_layout(sh1, st1, (B, M, N), (N * M, 1, M))
    want_fused = O.binary(O.MUL, s1, sh1, st1, 0, c, (B, M, N), (N * M, 1, M), 0, sh2, st2)
    kid = U.fusion_compile("in f32\nin f32\nin f32\nadd %0 %1\nmul %3 %2\nout %4\n")
    for cap in (1, 7):
        print(f"grid cap {cap}", flush=True)
        try:
            check(abi.lib.trs_debug_pointwise_grid_cap(cap))
            for name, (args, want) in cases.items():
                got = U.binary(*args)
                try:
                    assert_bitwise_equal(got, want)
                except AssertionError as e:
                    raise AssertionError(f"{name}, cap {cap}: {e}") from None
            devs = [U.dev(x) for x in (a, b, c)]
            out = U.out_buffer(B * M * N)
            U.fusion_launch(kid, devs, [layout_of((B, 1, N)), layout_of((1, M, N)), layout_of((B, M, N), (N * M, 1, M))],
                            out, layout_of((B, M, N)))
            assert_bitwise_equal(out.to_numpy(count=B * M * N), want_fused)
        finally:
            check(abi.lib.trs_debug_pointwise_grid_cap(0))

