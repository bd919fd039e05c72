"""HIP event timing on the library's own stream (trs_stream)."""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float, c_int, c_void_p

from .abi import check, lib

_hip = ctypes.CDLL("libamdhip64.so.7")
_hip.hipEventCreate.argtypes = [POINTER(c_void_p)]
_hip.hipEventCreate.restype = c_int
_hip.hipEventRecord.argtypes = [c_void_p, c_void_p]
_hip.hipEventRecord.restype = c_int
_hip.hipEventSynchronize.argtypes = [c_void_p]
_hip.hipEventSynchronize.restype = c_int
_hip.hipEventElapsedTime.argtypes = [POINTER(c_float), c_void_p, c_void_p]
_hip.hipEventElapsedTime.restype = c_int
_hip.hipEventDestroy.argtypes = [c_void_p]
_hip.hipEventDestroy.restype = c_int


def _ok(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed with HIP error {rc}")


def stream() -> c_void_p:
    s = c_void_p()
    check(lib.trs_stream(ctypes.byref(s)))
    return s


class Event:
    def __init__(self):
        self.ev = c_void_p()
        _ok(_hip.hipEventCreate(ctypes.byref(self.ev)), "hipEventCreate")

    def record(self, s: c_void_p) -> None:
        _ok(_hip.hipEventRecord(self.ev, s), "hipEventRecord")

    def synchronize(self) -> None:
        _ok(_hip.hipEventSynchronize(self.ev), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = c_float()
        _ok(_hip.hipEventElapsedTime(ctypes.byref(ms), self.ev, end.ev), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            if self.ev.value:
                _hip.hipEventDestroy(self.ev)
        except Exception:
            pass


def time_launches(fn, reps: int, warmup: int = 3) -> list[float]:
    """Per-call device time (ms) of `fn` (which enqueues work on trs_stream)."""
    s = stream()
    for _ in range(warmup):
        fn()
    check(lib.trs_synchronize())
    times = []
    evs = [(Event(), Event()) for _ in range(reps)]
    for a, b in evs:
        a.record(s)
        fn()
        b.record(s)
    for a, b in evs:
        b.synchronize()
        times.append(a.elapsed_ms(b))
    return times


def time_region(fn, reps: int, warmup: int = 3) -> float:
    """Average device time (ms) per call of `fn` over `reps` back-to-back calls,
    from one pair of events around the whole region on trs_stream."""
    s = stream()
    for _ in range(warmup):
        fn()
    check(lib.trs_synchronize())
    a, b = Event(), Event()
    a.record(s)
    for _ in range(reps):
        fn()
    b.record(s)
    b.synchronize()
    return a.elapsed_ms(b) / reps
