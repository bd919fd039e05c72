"""Host <-> device copies: ingest and egress of whole buffers.

Copies to the device from pageable memory of at least 16 MiB, and from the
device to pageable memory of at least 4 MiB, are pipelined through two
page-locked chunks of up to 16 MiB (at least four steps per copy);
page-locked memory (trs_host_alloc) goes as one DMA.  The sizes below
straddle both thresholds and every chunk boundary case (exactly one chunk,
one byte over, an odd number of chunks, a ragged tail), with host and device
addresses that are not 4-byte aligned.  All checks are byte-exact.
"""
import ctypes
import threading

import numpy as np
import pytest

import torch_rs
from trs_backend import abi
from trs_backend.abi import DeviceArray, check

pytestmark = pytest.mark.gpu

MIB = 1 << 20
SIZES = [1, 4095, 4 * MIB - 1, 4 * MIB, 16 * MIB - 1, 16 * MIB, 16 * MIB + 1, 3 * 16 * MIB, 2 * 16 * MIB + 12345, 100 * MIB + 7]


def _bytes(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("host_off,dev_off", [(0, 0), (3, 5)])
def test_pageable_round_trip_is_byte_exact(n, host_off, dev_off):
    src_buf = _bytes(n + host_off, n)
    src = src_buf[host_off:]
    d = DeviceArray(n + dev_off)
    dst_dev = ctypes.c_void_p(d.addr + dev_off)
    check(abi.lib.trs_memcpy_h2d(dst_dev, ctypes.c_void_p(src.ctypes.data), n))
    out_buf = np.zeros(n + host_off, np.uint8)
    out = out_buf[host_off:]
    check(abi.lib.trs_memcpy_d2h(ctypes.c_void_p(out.ctypes.data), dst_dev, n))
    assert np.array_equal(out, src)
    assert not out_buf[:host_off].any()  # nothing written before the destination


@pytest.mark.parametrize("n", [4095, 16 * MIB + 1, 40 * MIB + 3])
def test_pinned_round_trip_and_mixed_directions(n):
    p = ctypes.c_void_p()
    check(abi.lib.trs_host_alloc(n, ctypes.byref(p)))
    try:
        pin = np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(p.value))
        src = _bytes(n, 7)
        pin[:] = src
        d = DeviceArray(n)
        check(abi.lib.trs_memcpy_h2d(d.ptr, p, n))          # page-locked -> device
        back = np.empty(n, np.uint8)
        check(abi.lib.trs_memcpy_d2h(ctypes.c_void_p(back.ctypes.data), d.ptr, n))  # device -> pageable
        assert np.array_equal(back, src)
        pin[:] = 0
        check(abi.lib.trs_memcpy_d2h(p, d.ptr, n))          # device -> page-locked
        assert np.array_equal(pin, src)
        del pin
    finally:
        check(abi.lib.trs_host_free(p))


def test_host_alloc_of_zero_bytes_and_free_of_null():
    p = ctypes.c_void_p(1234)
    check(abi.lib.trs_host_alloc(0, ctypes.byref(p)))
    assert not p.value
    check(abi.lib.trs_host_free(None))


def test_concurrent_staged_copies_from_threads():
    """Threads share the device's two staging chunks; each copy must still
    see only its own bytes."""
    n = 20 * MIB + 9
    srcs = [_bytes(n, 100 + i) for i in range(4)]
    devs = [DeviceArray(n) for _ in srcs]
    errors = []
    barrier = threading.Barrier(4)

    def worker(i):
        try:
            barrier.wait()
            for _ in range(3):
                check(abi.lib.trs_memcpy_h2d(devs[i].ptr, ctypes.c_void_p(srcs[i].ctypes.data), n))
                out = np.empty(n, np.uint8)
                check(abi.lib.trs_memcpy_d2h(ctypes.c_void_p(out.ctypes.data), devs[i].ptr, n))
                if not np.array_equal(out, srcs[i]):
                    errors.append(f"thread {i}: bytes differ")
        except Exception as e:  # reported below
            errors.append(repr(e))

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors


def test_tensor_ingest_and_egress_through_numpy():
    rng = np.random.default_rng(3)
    a = rng.standard_normal((2049, 4099)).astype(np.float32)  # 33.6 MB: staged, ragged tail
    t = torch_rs.tensor(a, device="cuda")
    assert np.array_equal(t.numpy().view(np.uint32), a.view(np.uint32))
    # a transposed view is made contiguous on the device, then copied out
    assert np.array_equal(t.T.numpy(), a.T)
    assert np.array_equal(np.asarray(t[5]), a[5])


def test_pinned_arrays_through_torch_rs():
    a = torch_rs.cuda.empty_pinned((1024, 3000))
    assert a.dtype == np.float32 and a.shape == (1024, 3000) and a.flags.c_contiguous
    a[:] = np.random.default_rng(4).standard_normal(a.shape).astype(np.float32)
    t = torch_rs.tensor(a, device="cuda")
    out = torch_rs.cuda.empty_pinned((3000, 1024))
    torch_rs.cuda.copy_to_host(t.T, out)
    assert np.array_equal(out, a.T)
    m = torch_rs.cuda.empty_pinned(17, dtype=np.uint8)
    assert m.dtype == np.uint8 and m.shape == (17,)
    assert torch_rs.cuda.empty_pinned((0, 4)).shape == (0, 4)
    with pytest.raises(RuntimeError, match="shape"):
        torch_rs.cuda.copy_to_host(t, np.empty((3, 3), np.float32))
    with pytest.raises(RuntimeError, match="float32"):
        torch_rs.cuda.copy_to_host(t, np.empty((1024, 3000), np.float64))
    with pytest.raises(RuntimeError, match="C-contiguous"):
        torch_rs.cuda.copy_to_host(t, np.empty((3000, 1024), np.float32).T)
    with pytest.raises(RuntimeError, match="supports float32 and uint8"):
        torch_rs.cuda.empty_pinned(4, dtype=np.float64)
