"""Helpers for GPU parity tests: device buffers and C-ABI calls by layout."""
from __future__ import annotations

import ctypes

import numpy as np

import oracle as O
from trs_backend import abi
from trs_backend.abi import DeviceArray, check, layout_of


def dev(arr: np.ndarray) -> DeviceArray:
    arr = np.ascontiguousarray(arr)
    if arr.nbytes == 0:
        arr = np.zeros(1, dtype=arr.dtype)
    return DeviceArray.from_numpy(arr)


def out_buffer(n: int, fill=np.nan) -> DeviceArray:
    return dev(np.full(max(n, 1), fill, np.float32))


def storage_size(shape, strides, offset=0) -> int:
    return O.storage_size(tuple(shape), tuple(strides), offset)


def binary(op, a, ashape, astr, aoff, b, bshape, bstr, boff, oshape, ostr):
    da, db = dev(a), dev(b)
    n = storage_size(oshape, ostr)
    do = out_buffer(n)
    check(abi.lib.trs_binary_f32(op, da.ptr, ctypes.byref(layout_of(ashape, astr, aoff)), db.ptr,
                                 ctypes.byref(layout_of(bshape, bstr, boff)), do.ptr,
                                 ctypes.byref(layout_of(oshape, ostr))))
    return do.to_numpy(count=n)


def scalar(op, a, shape, strides, off, s, ostr):
    da = dev(a)
    n = storage_size(shape, ostr)
    do = out_buffer(n)
    check(abi.lib.trs_binary_scalar_f32(op, da.ptr, ctypes.byref(layout_of(shape, strides, off)), ctypes.c_float(s),
                                        do.ptr, ctypes.byref(layout_of(shape, ostr))))
    return do.to_numpy(count=n)


def unary(op, a, shape, strides, off, ostr):
    da = dev(a)
    n = storage_size(shape, ostr)
    do = out_buffer(n)
    check(abi.lib.trs_unary_f32(op, da.ptr, ctypes.byref(layout_of(shape, strides, off)), do.ptr,
                                ctypes.byref(layout_of(shape, ostr))))
    return do.to_numpy(count=n)


def matmul(a, ashape, astr, aoff, b, bshape, bstr, boff):
    da, db = dev(a), dev(b)
    r = len(ashape)
    oshape = tuple(ashape[:-1]) + (bshape[-1],)
    n = int(np.prod(oshape))
    do = out_buffer(n)
    check(abi.lib.trs_matmul_f32(da.ptr, ctypes.byref(layout_of(ashape, astr, aoff)), db.ptr,
                                 ctypes.byref(layout_of(bshape, bstr, boff)), do.ptr,
                                 ctypes.byref(layout_of(oshape))))
    del r
    return do.to_numpy(count=n).reshape(oshape)


def fusion_compile(ir: str) -> int:
    kid = ctypes.c_uint64()
    check(abi.lib.trs_fusion_compile(ir.encode(), len(ir), ctypes.byref(kid)))
    return kid.value


def fusion_launch(kid: int, inputs, layouts, out: DeviceArray, olayout) -> None:
    n = len(inputs)
    ptrs = (ctypes.c_void_p * n)(*[x.addr for x in inputs])
    lays = (abi.Layout * n)(*layouts)
    check(abi.lib.trs_fusion_launch(kid, n, ptrs, lays, out.ptr, ctypes.byref(olayout)))


def fusion_launch_multi(kid: int, inputs, layouts, outs, olayout) -> int:
    """trs_fusion_launch_multi; returns the status code (not checked)."""
    n, m = len(inputs), len(outs)
    ptrs = (ctypes.c_void_p * n)(*[x.addr for x in inputs])
    lays = (abi.Layout * n)(*layouts)
    optrs = (ctypes.c_void_p * m)(*[o.addr for o in outs])
    return abi.lib.trs_fusion_launch_multi(kid, n, ptrs, lays, m, optrs, ctypes.byref(olayout))


def special_mix(rng, n: int) -> np.ndarray:
    """Normals with IEEE specials sprinkled in (signed zeros, infs, NaNs, subnormals)."""
    x = rng.standard_normal(n).astype(np.float32)
    if n >= 16:
        specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 1e-39, -3e38, 3e38],
                            dtype=np.float32)
        idx = rng.choice(n, size=min(n // 8, 64), replace=False)
        x[idx] = specials[rng.integers(0, len(specials), size=idx.size)]
    return x
