"""Shared helpers for the parity tests (bit patterns, ulp distances, fixtures)."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def golden(name: str = "reference_vectors.json") -> dict:
    return json.loads((GOLDEN / name).read_text())


def f32_from_bits(bits) -> np.ndarray:
    return np.array([int(b, 16) if isinstance(b, str) else int(b) for b in bits], dtype=np.uint32).view(np.float32)


def bits_of(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32)


def check_bits(actual, expected_spec) -> None:
    """expected_spec: list of '0x...' bit strings or 'nan'."""
    actual = np.asarray(actual, dtype=np.float32)
    assert actual.size == len(expected_spec), (actual.size, len(expected_spec))
    for i, (a, e) in enumerate(zip(actual, expected_spec)):
        if e == "nan":
            assert np.isnan(a), f"element {i}: expected NaN, got {a!r}"
        else:
            got = int(np.float32(a).view(np.uint32))
            assert got == int(e, 16), f"element {i}: expected {e}, got {got:#010x} ({a!r})"


def assert_bitwise_equal(actual, expected, nan_equal: bool = True) -> None:
    """Bit-exact equality; all NaNs compare equal when nan_equal (payloads differ by ISA)."""
    a = np.ascontiguousarray(np.asarray(actual, dtype=np.float32)).reshape(-1)
    e = np.ascontiguousarray(np.asarray(expected, dtype=np.float32)).reshape(-1)
    assert a.shape == e.shape, (a.shape, e.shape)
    ab, eb = a.view(np.uint32), e.view(np.uint32)
    same = ab == eb
    if nan_equal:
        same |= np.isnan(a) & np.isnan(e)
    if not same.all():
        idx = np.flatnonzero(~same)[:8]
        detail = ", ".join(f"[{i}] got {ab[i]:#010x} ({a[i]!r}) want {eb[i]:#010x} ({e[i]!r})" for i in idx)
        raise AssertionError(f"{(~same).sum()} of {a.size} elements differ: {detail}")


def ordered_int(x: np.ndarray) -> np.ndarray:
    """Map float32 to integers whose difference counts representable floats."""
    i = np.ascontiguousarray(x, dtype=np.float32).view(np.int32).astype(np.int64)
    return np.where(i < 0, -(i & 0x7FFFFFFF), i)


def ulp_distance(a, b) -> np.ndarray:
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    d = np.abs(ordered_int(a) - ordered_int(b))
    both_nan = np.isnan(a) & np.isnan(b)
    return np.where(both_nan, 0, d)


def ulp_of(x) -> np.ndarray:
    """Spacing of float32 at |x| (np.spacing of the magnitude)."""
    return np.spacing(np.abs(np.asarray(x, dtype=np.float32))).astype(np.float64)
