"""ctypes declarations for every entry point of include/trs_hip.h.

Loading fails loudly when the library has not been built: there is no CPU
fallback anywhere in the product path.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_uint32, \
    c_uint64, c_void_p
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent.parent
LIB_DIR = PKG / "lib"
MAX_RANK = 25

TRS_ADD, TRS_SUB, TRS_MUL, TRS_DIV = 0, 1, 2, 3
TRS_S_ADD, TRS_S_SUB, TRS_S_MUL, TRS_S_DIV, TRS_S_RSUB, TRS_S_RDIV = range(6)
TRS_EXP, TRS_RELU, TRS_NEG, TRS_COPY = 0, 1, 2, 3
TRS_E_SHAPE_MISMATCH, TRS_E_INVALID_ARGUMENT, TRS_E_FUSION = -4, -7, -9

ERROR_NAMES = {
    -1: "ALLOCATION_FAILED", -2: "INDEX_OVERFLOW", -3: "STRIDE_OVERFLOW", -4: "SHAPE_MISMATCH",
    -5: "MATMUL_INNER_MISMATCH", -6: "MATMUL_REQUIRES_MATRICES", -7: "INVALID_ARGUMENT", -8: "HIP",
    -9: "FUSION", -10: "NO_DEVICE",
}


class Layout(ctypes.Structure):
    _fields_ = [
        ("rank", c_int32),
        ("reserved", c_int32),
        ("shape", c_int64 * MAX_RANK),
        ("stride", c_int64 * MAX_RANK),
        ("offset", c_int64),
    ]

    def dims(self):
        return tuple(self.shape[i] for i in range(self.rank))

    def strides(self):
        return tuple(self.stride[i] for i in range(self.rank))


class TrsError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {message}")
        self.code = code
        self.message = message


def contiguous_strides(shape) -> tuple:
    strides, s = [], 1
    for d in reversed(shape):
        strides.append(s)
        s *= max(int(d), 1)
    return tuple(reversed(strides))


def layout_of(shape, strides=None, offset: int = 0) -> Layout:
    shape = tuple(int(d) for d in shape)
    if len(shape) > MAX_RANK:
        raise ValueError(f"rank above {MAX_RANK}")
    if strides is None:
        strides = contiguous_strides(shape)
    lay = Layout()
    lay.rank = len(shape)
    for i, (d, s) in enumerate(zip(shape, strides)):
        lay.shape[i] = d
        lay.stride[i] = int(s)
    lay.offset = int(offset)
    return lay


class PwPlanInfo(ctypes.Structure):
    """trs_pw_plan_info: the launch plan trs_pointwise_plan reports."""
    _fields_ = [
        ("variant", c_int32),     # 0 nothing to do, 1 flat, 2 rows, 3 transposing, 4 generic
        ("rank", c_int32),
        ("vec", c_int32),
        ("fixed_rank", c_int32),
        ("skew", c_int32),
        ("walk", c_int32),
        ("trans", c_uint32),
        ("held", c_uint32),
        ("once", c_uint32),
        ("block", c_int32),
        ("grid", ctypes.c_int64),
        ("split", c_int32),       # dims walked on the host (the fewest indices), one launch each
        ("launches", c_int32),    # kernel launches per call (saturates at INT32_MAX)
    ]


_LP = POINTER(Layout)
_FP = POINTER(c_float)

_SIGNATURES = {
    "trs_init": ([], c_int),
    "trs_device_count": ([POINTER(c_int)], c_int),
    "trs_set_device": ([c_int], c_int),
    "trs_get_device": ([POINTER(c_int)], c_int),
    "trs_device_info": ([ctypes.c_char_p, c_size_t, POINTER(c_int), POINTER(c_int)], c_int),
    "trs_alloc": ([c_size_t, POINTER(c_void_p)], c_int),
    "trs_free": ([c_void_p], c_int),
    "trs_empty_cache": ([], c_int),
    "trs_host_alloc": ([c_size_t, POINTER(c_void_p)], c_int),
    "trs_host_free": ([c_void_p], c_int),
    "trs_memory_stats": ([POINTER(c_size_t), POINTER(c_size_t)], c_int),
    "trs_memcpy_h2d": ([c_void_p, c_void_p, c_size_t], c_int),
    "trs_memcpy_d2h": ([c_void_p, c_void_p, c_size_t], c_int),
    "trs_debug_fail_allocs_after": ([c_int64], c_int),
    "trs_debug_pointwise_grid_cap": ([c_int64], c_int),
    "trs_memcpy_d2d": ([c_void_p, c_void_p, c_size_t], c_int),
    "trs_memset_zero": ([c_void_p, c_size_t], c_int),
    "trs_synchronize": ([], c_int),
    "trs_stream": ([POINTER(c_void_p)], c_int),
    "trs_last_error": ([], c_char_p),
    "trs_binary_f32": ([c_int, c_void_p, _LP, c_void_p, _LP, c_void_p, _LP], c_int),
    "trs_binary_scalar_f32": ([c_int, c_void_p, _LP, c_float, c_void_p, _LP], c_int),
    "trs_unary_f32": ([c_int, c_void_p, _LP, c_void_p, _LP], c_int),
    "trs_mask_apply_f32": ([c_void_p, _LP, c_void_p, _LP, c_float, c_void_p, _LP], c_int),
    "trs_sum_f32": ([c_void_p, _LP, c_void_p], c_int),
    "trs_sum_f32_noalloc": ([c_void_p, _LP, c_void_p], c_int),
    "trs_fill_from_device_f32": ([c_void_p, c_size_t, c_void_p], c_int),
    "trs_fill_f32": ([c_void_p, c_size_t, c_float], c_int),
    "trs_mask_backward_f32": ([c_void_p, _LP, c_void_p, _LP, c_float, c_void_p, _LP], c_int),
    "trs_relu_backward_f32": ([c_void_p, _LP, c_void_p, c_void_p], c_int),
    "trs_mul_backward_f32": ([c_void_p, _LP, c_void_p, _LP, _LP, c_void_p], c_int),
    "trs_reduce_to_shape_f32": ([c_void_p, _LP, _LP, c_void_p], c_int),
    "trs_accumulate_f32": ([c_void_p, c_void_p, c_size_t], c_int),
    "trs_matmul_f32": ([c_void_p, _LP, c_void_p, _LP, c_void_p, _LP], c_int),
    "trs_matmul_plan_f32": ([c_void_p, _LP, c_void_p, _LP, c_void_p, _LP, POINTER(c_int), POINTER(c_int),
                             POINTER(c_int), POINTER(ctypes.c_int64), POINTER(ctypes.c_int64)], c_int),
    "trs_pointwise_plan": ([c_int, POINTER(c_void_p), POINTER(_LP), POINTER(c_int), c_void_p, _LP, c_int, c_int,
                            POINTER(PwPlanInfo)], c_int),
    "trs_fusion_compile": ([c_char_p, c_size_t, POINTER(c_uint64)], c_int),
    "trs_fusion_launch": ([c_uint64, c_int, POINTER(c_void_p), _LP, c_void_p, _LP], c_int),
    "trs_fusion_launch_multi": ([c_uint64, c_int, POINTER(c_void_p), _LP, c_int, POINTER(c_void_p), _LP], c_int),
    "trs_fusion_outputs": ([c_uint64, POINTER(c_int)], c_int),
    "trs_fusion_source": ([c_uint64, ctypes.c_char_p, c_size_t, POINTER(c_size_t)], c_int),
    "trs_fusion_compile_ms": ([c_uint64, POINTER(c_double)], c_int),
    "trs_fusion_from_disk_cache": ([c_uint64, POINTER(c_int)], c_int),
}


def _load(name: str) -> ctypes.CDLL:
    path = LIB_DIR / name
    if not path.exists():
        raise ImportError(f"{path} is not built; run `python pytorch-rs_amd/build.py`")
    return ctypes.CDLL(str(path))


lib = _load("libtrs_hip.so")
for _name, (_args, _res) in _SIGNATURES.items():
    _fn = getattr(lib, _name)
    _fn.argtypes = _args
    _fn.restype = _res

inputs_lib = _load("libtrs_inputs.so")
inputs_lib.trs_philox4x32_10.argtypes = [POINTER(c_uint32), POINTER(c_uint32), POINTER(c_uint32)]
inputs_lib.trs_philox4x32_10.restype = None
for _n in ("trs_gen_uniform_f32", "trs_gen_normal_f32"):
    getattr(inputs_lib, _n).argtypes = [c_uint64, c_uint32, c_double, c_double, c_void_p, c_uint64, c_int]
    getattr(inputs_lib, _n).restype = c_int
inputs_lib.trs_gen_mask_u8.argtypes = [c_uint64, c_uint32, c_double, c_void_p, c_uint64, c_int]
inputs_lib.trs_gen_mask_u8.restype = c_int


def check(rc: int) -> None:
    if rc != 0:
        msg = lib.trs_last_error()
        raise TrsError(rc, msg.decode() if msg else "")


def pointwise_plan(layouts, out_layout, bases=None, out=0x10000000000, elem_bytes=None, cu_count=256,
                   roles=False) -> PwPlanInfo:
    """trs_pointwise_plan for input `layouts` and `out_layout` (no device
    needed).  `bases` and `out` are addresses, used only for alignment and
    the overlap checks: by default far apart and 256-byte aligned."""
    n = len(layouts)
    if bases is None:
        bases = [0x20000000000 + i * 0x10000000000 for i in range(n)]
    ptrs = (c_void_p * n)(*bases)
    lays = (_LP * n)(*[ctypes.pointer(l) for l in layouts])
    eb = (c_int * n)(*(elem_bytes or [4] * n))
    info = PwPlanInfo()
    check(lib.trs_pointwise_plan(n, ptrs, lays, eb, c_void_p(out), ctypes.byref(out_layout), cu_count,
                                 1 if roles else 0, ctypes.byref(info)))
    return info


def device_count() -> int:
    n = c_int(0)
    rc = lib.trs_device_count(ctypes.byref(n))
    return n.value if rc == 0 else 0


def synchronize() -> None:
    check(lib.trs_synchronize())


class DeviceArray:
    """A raw HBM allocation (float32 or uint8) owned by Python."""

    def __init__(self, nbytes: int):
        self.ptr = c_void_p()
        self.nbytes = int(nbytes)
        check(lib.trs_alloc(self.nbytes, ctypes.byref(self.ptr)))

    @classmethod
    def from_numpy(cls, arr: np.ndarray) -> "DeviceArray":
        arr = np.ascontiguousarray(arr)
        d = cls(arr.nbytes)
        if arr.nbytes:
            check(lib.trs_memcpy_h2d(d.ptr, arr.ctypes.data, arr.nbytes))
        return d

    def to_numpy(self, dtype=np.float32, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else int(count)
        out = np.empty(n, dtype=dtype)
        if n:
            check(lib.trs_memcpy_d2h(out.ctypes.data, self.ptr, n * dtype.itemsize))
        return out

    @property
    def addr(self) -> int:
        return self.ptr.value or 0

    def free(self) -> None:
        if self.ptr.value:
            check(lib.trs_free(self.ptr))
            self.ptr = c_void_p()

    def __del__(self):
        try:
            if self.ptr.value:
                lib.trs_free(self.ptr)
        except Exception:
            pass


def gen_uniform(seed: int, stream: int, lo: float, hi: float, n: int, threads: int = 8) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    inputs_lib.trs_gen_uniform_f32(seed, stream, lo, hi, out.ctypes.data, n, threads)
    return out


def gen_normal(seed: int, stream: int, mean: float, std: float, n: int, threads: int = 8) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    inputs_lib.trs_gen_normal_f32(seed, stream, mean, std, out.ctypes.data, n, threads)
    return out


def gen_mask(seed: int, stream: int, keep: float, n: int, threads: int = 8) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    inputs_lib.trs_gen_mask_u8(seed, stream, keep, out.ctypes.data, n, threads)
    return out


def philox(ctr, key) -> tuple:
    c = (c_uint32 * 4)(*ctr)
    k = (c_uint32 * 2)(*key)
    o = (c_uint32 * 4)()
    inputs_lib.trs_philox4x32_10(c, k, o)
    return tuple(o)
