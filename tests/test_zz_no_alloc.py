"""trs_sum_f32_noalloc: the sum entry point that allocates nothing.

Its block partials live in a static device array instead of a block-cache
buffer; otherwise it runs trs_sum_f32's kernels, so its results must equal
trs_sum_f32's bit for bit.  Two calls in a row, the second on a smaller
input, check that the partials the first call left in the shared array do
not leak into the second.  The library's block cache must neither grow nor
be drawn from across the calls.
"""
import ctypes

import numpy as np
import pytest

from trs_backend import abi
from trs_backend.abi import DeviceArray, check, layout_of

pytestmark = pytest.mark.gpu


def _stats():
    live, cached = ctypes.c_size_t(), ctypes.c_size_t()
    check(abi.lib.trs_memory_stats(ctypes.byref(live), ctypes.byref(cached)))
    return live.value, cached.value


def _sum(fn, x: DeviceArray, lay, out: DeviceArray) -> np.uint32:
    check(fn(x.ptr, ctypes.byref(lay), out.ptr))
    return out.to_numpy(count=1).view(np.uint32)[0]


def test_noalloc_sum_equals_the_allocating_sum_and_allocates_nothing():
    check(abi.lib.trs_init())
    rng = np.random.default_rng(2024)
    # (elements, layout): two-pass (1,024 partials), two-pass with fewer
    # partials, a strided two-pass view, the one-block path, all -0.0, empty.
    big = rng.standard_normal(3_000_017).astype(np.float32) + np.float32(0.25)
    small = rng.standard_normal(100_003).astype(np.float32)
    tall = rng.standard_normal(600 * 301).astype(np.float32)
    tiny = rng.standard_normal(20_000).astype(np.float32)
    zeros = np.full(50_000, -0.0, np.float32)
    cases = [
        (big, layout_of((big.size,))),
        (small, layout_of((small.size,))),
        (tall, layout_of((301, 600), (1, 301))),  # a transposed view: decoded in logical order
        (tiny, layout_of((tiny.size,))),
        (zeros, layout_of((zeros.size,))),
        (np.zeros(1, np.float32), layout_of((0, 5))),
    ]
    devs = [DeviceArray.from_numpy(x) for x, _ in cases]
    out_ref, out_na = DeviceArray(4), DeviceArray(4)
    check(abi.lib.trs_synchronize())
    check(abi.lib.trs_empty_cache())
    before = _stats()
    assert before[1] == 0

    got = []
    for (x, lay), d in zip(cases, devs):
        got.append(_sum(abi.lib.trs_sum_f32_noalloc, d, lay, out_na))
    assert _stats() == before, "the no-allocation sum took memory from the block cache"

    for (x, lay), d, g in zip(cases, devs, got):
        want = _sum(abi.lib.trs_sum_f32, d, lay, out_ref)
        assert g == want, (x.size, hex(g), hex(want))
    assert got[4] == 0x80000000 and got[5] == 0x80000000  # -0.0: all-(-0.0) and empty
    # The allocating entry point does draw a partials buffer from the cache,
    # so the stats check above would have seen one.
    assert _stats()[1] > 0

    # The two calls again in reverse size order (smaller second), interleaved
    # with the allocating sum, after the cache was refilled.
    for i in (0, 1):
        assert _sum(abi.lib.trs_sum_f32_noalloc, devs[i], cases[i][1], out_na) == got[i]
        assert _sum(abi.lib.trs_sum_f32, devs[i], cases[i][1], out_ref) == got[i]


def test_noalloc_sum_rejects_bad_arguments_like_the_allocating_sum():
    check(abi.lib.trs_init())
    x = DeviceArray.from_numpy(np.ones(40_000, np.float32))
    lay = layout_of((40_000,))
    assert abi.lib.trs_sum_f32_noalloc(x.ptr, ctypes.byref(lay), None) == abi.lib.trs_sum_f32(
        x.ptr, ctypes.byref(lay), None) == -7
    bad = layout_of((40_000,), (-1,))
    out = DeviceArray(4)
    assert abi.lib.trs_sum_f32_noalloc(x.ptr, ctypes.byref(bad), out.ptr) == -7
