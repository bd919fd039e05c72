"""ctypes wrapper of liboracle.so -- TEST INFRASTRUCTURE ONLY.

The CPU restatement of the reference hot path (trs_oracle.c).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module,
and only as the checker (or the timed CPU baseline), never as a product path.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
MAX_RANK = 25


class OLayout(ctypes.Structure):
    _fields_ = [
        ("rank", c_int32),
        ("reserved", c_int32),
        ("shape", c_int64 * MAX_RANK),
        ("stride", c_int64 * MAX_RANK),
        ("offset", c_int64),
    ]


def contiguous_strides(shape):
    strides, s = [], 1
    for d in reversed(shape):
        strides.append(s)
        s *= max(int(d), 1)
    return tuple(reversed(strides))


def olayout(shape, strides=None, offset=0) -> OLayout:
    shape = tuple(int(d) for d in shape)
    if strides is None:
        strides = contiguous_strides(shape)
    lay = OLayout()
    lay.rank = len(shape)
    for i, (d, s) in enumerate(zip(shape, strides)):
        lay.shape[i] = d
        lay.stride[i] = int(s)
    lay.offset = int(offset)
    return lay


_LP = POINTER(OLayout)
_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            raise ImportError(f"{path} not built; run `make -C oracle`")
        L = ctypes.CDLL(str(path))
        sig = {
            "orc_libc_version": ([], c_char_p),
            "orc_contiguous_strides": ([c_int, c_void_p, c_void_p], c_int),
            "orc_layout_is_contiguous": ([c_int, c_void_p, c_void_p, c_uint64], c_int),
            "orc_is_non_overlapping_and_dense": ([c_int, c_void_p, c_void_p, c_uint64], c_int),
            "orc_is_channels_last_contiguous": ([c_int, c_void_p, c_void_p], c_int),
            "orc_elementwise_output_strides": ([c_int, c_void_p, c_int, _LP, c_void_p], c_int),
            "orc_unary_output_strides": ([_LP, c_void_p], c_int),
            "orc_scalar_output_strides": ([_LP, c_void_p], c_int),
            "orc_binary_output_layout": ([_LP, _LP, _LP], c_int),
            "orc_binary_f32": ([c_int, c_void_p, _LP, c_void_p, _LP, c_void_p, _LP], c_int),
            "orc_scalar_f32": ([c_int, c_void_p, _LP, c_float, c_void_p, _LP], c_int),
            "orc_unary_f32": ([c_int, c_void_p, _LP, c_void_p, _LP], c_int),
            "orc_unary_contig_f32": ([c_int, c_void_p, c_void_p, c_uint64], None),
            "orc_binary_contig_f32": ([c_int, c_void_p, c_void_p, c_void_p, c_uint64], None),
            "orc_scalar_contig_f32": ([c_int, c_void_p, c_float, c_void_p, c_uint64], None),
            "orc_row_broadcast_f32": ([c_int, c_void_p, c_void_p, c_void_p, c_uint64, c_uint64], None),
            "orc_mask_apply_f32": ([c_void_p, c_void_p, c_float, c_void_p, c_uint64], None),
            "orc_sum_f32": ([c_void_p, _LP], c_float),
            "orc_sum_abs_f64": ([c_void_p, c_uint64], c_double),
            "orc_matmul_f32": ([c_void_p, _LP, c_void_p, _LP, c_void_p, c_int64, c_int64, c_int64], c_int),
            "orc_matmul_row_blocked_f32": ([c_void_p, c_void_p, c_void_p, c_uint64, c_uint64, c_uint64], None),
            "orc_matmul_row_blocked_threads_f32": ([c_void_p, c_void_p, c_void_p, c_uint64, c_uint64, c_uint64,
                                                    c_int], None),
            "orc_matmul_rows_f32": ([c_void_p, _LP, c_void_p, _LP, c_void_p, c_int64, c_void_p], c_int),
            "orc_matmul_abs_rows_f64": ([c_void_p, _LP, c_void_p, _LP, c_void_p, c_int64, c_void_p], c_int),
            "orc_relu_backward_f32": ([c_void_p, _LP, c_void_p, c_void_p], None),
            "orc_mul_backward_f32": ([c_void_p, _LP, c_void_p, _LP, _LP, c_void_p], None),
            "orc_reduce_to_shape_f32": ([c_void_p, _LP, _LP, c_void_p], None),
            "orc_permute_backward_f32": ([c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p], None),
            "orc_accumulate_f32": ([c_void_p, c_void_p, c_uint64], None),
            "orc_exp_max_ulp": ([c_void_p, c_uint32, c_uint64, c_int, POINTER(c_uint64)], c_uint64),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


ADD, SUB, MUL, DIV = 0, 1, 2, 3
S_ADD, S_SUB, S_MUL, S_DIV, S_RSUB, S_RDIV = range(6)
EXP, RELU, NEG, COPY = 0, 1, 2, 3


class OracleError(RuntimeError):
    pass


def _chk(rc):
    if rc != 0:
        raise OracleError(rc)


def _u64(vals):
    return np.asarray(vals, dtype=np.uint64)


def libc_version() -> str:
    return lib().orc_libc_version().decode()


def contiguous(shape):
    out = np.zeros(max(len(shape), 1), dtype=np.uint64)
    sh = _u64(shape or [0])
    _chk(lib().orc_contiguous_strides(len(shape), _p(sh), _p(out)))
    return tuple(int(v) for v in out[: len(shape)])


def is_contiguous(shape, strides) -> bool:
    n = int(np.prod(np.asarray(shape, dtype=object))) if shape else 1
    sh, st = _u64(shape or [0]), _u64(strides or [0])
    return bool(lib().orc_layout_is_contiguous(len(shape), _p(sh), _p(st), n % (1 << 64)))


def is_non_overlapping_and_dense(shape, strides) -> bool:
    n = int(np.prod(np.asarray(shape, dtype=object))) if shape else 1
    sh, st = _u64(shape or [0]), _u64(strides or [0])
    return bool(lib().orc_is_non_overlapping_and_dense(len(shape), _p(sh), _p(st), n % (1 << 64)))


def unary_output_strides(shape, strides):
    out = np.zeros(MAX_RANK, dtype=np.int64)
    _chk(lib().orc_unary_output_strides(ctypes.byref(olayout(shape, strides)), _p(out)))
    return tuple(int(v) for v in out[: len(shape)])


def scalar_output_strides(shape, strides):
    out = np.zeros(MAX_RANK, dtype=np.int64)
    _chk(lib().orc_scalar_output_strides(ctypes.byref(olayout(shape, strides)), _p(out)))
    return tuple(int(v) for v in out[: len(shape)])


def binary_output_layout(lshape, lstrides, rshape, rstrides):
    out = OLayout()
    _chk(lib().orc_binary_output_layout(ctypes.byref(olayout(lshape, lstrides)),
                                        ctypes.byref(olayout(rshape, rstrides)), ctypes.byref(out)))
    return tuple(out.shape[i] for i in range(out.rank)), tuple(out.stride[i] for i in range(out.rank))


def storage_size(shape, strides, offset=0) -> int:
    if any(d == 0 for d in shape):
        return offset
    return offset + 1 + sum((d - 1) * s for d, s in zip(shape, strides))


def binary(op, lbuf, lshape, lstrides, loff, rbuf, rshape, rstrides, roff, oshape, ostrides):
    n = storage_size(oshape, ostrides)
    out = np.zeros(max(n, 1), dtype=np.float32)
    _chk(lib().orc_binary_f32(op, _p(lbuf), ctypes.byref(olayout(lshape, lstrides, loff)), _p(rbuf),
                              ctypes.byref(olayout(rshape, rstrides, roff)), _p(out),
                              ctypes.byref(olayout(oshape, ostrides))))
    return out[:n]


def scalar(op, buf, shape, strides, off, s, ostrides):
    n = storage_size(shape, ostrides)
    out = np.zeros(max(n, 1), dtype=np.float32)
    _chk(lib().orc_scalar_f32(op, _p(buf), ctypes.byref(olayout(shape, strides, off)), c_float(s), _p(out),
                              ctypes.byref(olayout(shape, ostrides))))
    return out[:n]


def unary(op, buf, shape, strides, off, ostrides):
    n = storage_size(shape, ostrides)
    out = np.zeros(max(n, 1), dtype=np.float32)
    _chk(lib().orc_unary_f32(op, _p(buf), ctypes.byref(olayout(shape, strides, off)), _p(out),
                             ctypes.byref(olayout(shape, ostrides))))
    return out[:n]


def unary_contig(op, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_unary_contig_f32(op, _p(x), _p(out), x.size)
    return out


def binary_contig(op, a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty_like(a)
    lib().orc_binary_contig_f32(op, _p(a), _p(b), _p(out), a.size)
    return out


def scalar_contig(op, a, s):
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty_like(a)
    lib().orc_scalar_contig_f32(op, _p(a), c_float(s), _p(out), a.size)
    return out


def row_broadcast(op, x, v, rows, cols):
    out = np.empty(rows * cols, dtype=np.float32)
    lib().orc_row_broadcast_f32(op, _p(x), _p(v), _p(out), rows, cols)
    return out


def mask_apply(h, mask, s):
    out = np.empty_like(h)
    lib().orc_mask_apply_f32(_p(h), _p(mask), c_float(s), _p(out), h.size)
    return out


def sum_f32(buf, shape, strides=None, off=0) -> np.float32:
    return np.float32(lib().orc_sum_f32(_p(buf), ctypes.byref(olayout(shape, strides, off))))


def sum_abs(buf) -> float:
    buf = np.ascontiguousarray(buf, dtype=np.float32)
    return float(lib().orc_sum_abs_f64(_p(buf), buf.size))


def matmul(a, ashape, astrides, aoff, b, bshape, bstrides, boff, batch=1, bsa=0, bsb=0):
    M, N = ashape[0], bshape[1]
    out = np.zeros(max(batch * M * N, 1), dtype=np.float32)
    _chk(lib().orc_matmul_f32(_p(a), ctypes.byref(olayout(ashape, astrides, aoff)), _p(b),
                              ctypes.byref(olayout(bshape, bstrides, boff)), _p(out), batch, bsa, bsb))
    return out[: batch * M * N]


def matmul_rows(a, ashape, astrides, b, bshape, bstrides, rows):
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    N = bshape[1]
    out = np.zeros(len(rows) * N, dtype=np.float32)
    bound = np.zeros(len(rows) * N, dtype=np.float64)
    la, lb = olayout(ashape, astrides), olayout(bshape, bstrides)
    _chk(lib().orc_matmul_rows_f32(_p(a), ctypes.byref(la), _p(b), ctypes.byref(lb), _p(rows), len(rows), _p(out)))
    _chk(lib().orc_matmul_abs_rows_f64(_p(a), ctypes.byref(la), _p(b), ctypes.byref(lb), _p(rows), len(rows),
                                       _p(bound)))
    return out.reshape(len(rows), N), bound.reshape(len(rows), N)


def relu_backward(inp, shape, strides, off, up):
    n = int(np.prod(shape)) if shape else 1
    out = np.zeros(max(n, 1), dtype=np.float32)
    lib().orc_relu_backward_f32(_p(inp), ctypes.byref(olayout(shape, strides, off)), _p(up), _p(out))
    return out[:n]


def mul_backward(up, oshape, other, other_shape, other_strides, other_off, self_shape):
    n = int(np.prod(self_shape)) if self_shape else 1
    out = np.zeros(max(n, 1), dtype=np.float32)
    lib().orc_mul_backward_f32(_p(up), ctypes.byref(olayout(oshape)), _p(other),
                               ctypes.byref(olayout(other_shape, other_strides, other_off)),
                               ctypes.byref(olayout(self_shape)), _p(out))
    return out[:n]


def reduce_to_shape(up, oshape, self_shape):
    n = int(np.prod(self_shape)) if self_shape else 1
    out = np.zeros(max(n, 1), dtype=np.float32)
    lib().orc_reduce_to_shape_f32(_p(up), ctypes.byref(olayout(oshape)), ctypes.byref(olayout(self_shape)), _p(out))
    return out[:n]


def permute_backward(up, out_shape, dims, in_shape):
    n = int(np.prod(in_shape)) if in_shape else 1
    out = np.zeros(max(n, 1), dtype=np.float32)
    os_, d_, is_ = (np.asarray(v, dtype=np.int64) for v in (out_shape, dims, in_shape))
    lib().orc_permute_backward_f32(_p(up), len(out_shape), _p(os_), _p(d_), _p(is_), _p(out))
    return out[:n]


def exp_max_ulp(got: np.ndarray, first_bits: int, threads: int = 8):
    """(max ulp distance, index) of got[i] from glibc expf(bits first_bits + i)."""
    got = np.ascontiguousarray(got, dtype=np.float32)
    idx = c_uint64()
    worst = lib().orc_exp_max_ulp(_p(got), first_bits, got.size, threads, ctypes.byref(idx))
    return int(worst), int(idx.value)


def matmul_threads(a: np.ndarray, b: np.ndarray, threads: int = 16) -> np.ndarray:
    """Contiguous [M,K] @ [K,N] in the reference's order (k ascending from
    +0.0 per element), the row-blocked loop split over threads by output rows;
    bit-identical to matmul_row_blocked."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    out = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_row_blocked_threads_f32(_p(a), _p(b), _p(out), m, k, n, threads)
    return out


def matmul_row_blocked(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Contiguous [M,K] @ [K,N] with the reference's 4-row blocked loop."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    m, k = a.shape
    _, n = b.shape
    out = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_row_blocked_f32(_p(a), _p(b), _p(out), m, k, n)
    return out
