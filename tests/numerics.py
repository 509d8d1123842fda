"""Comparators of the reference's test support (tests/test_utils.hpp:37-227).

compare_close        |a - e| <= atol + rtol * |e|, non-finite values fail unless
                     both are the same infinity (test_utils.hpp:88-133).
compare_close_scaled |a - e| <= atol + rtol * scale, scale = sum |terms| of the
                     reduction (test_utils.hpp:149-190); any non-finite fails.
require_exact        bitwise equality (test_utils.hpp:218-227).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


class TestFailure(AssertionError):
    """A failed check (test_utils.hpp:24-27), distinct from library errors."""

    __test__ = False


@dataclass
class Comparison:
    matched: bool = True
    index: int = 0
    actual: float = 0.0
    expected: float = 0.0
    absolute_difference: float = 0.0
    relative_difference: float = 0.0
    worst_relative_difference: float = 0.0
    worst_index: int = 0
    non_finite: bool = False

    def __bool__(self) -> bool:
        return self.matched

    def describe(self) -> str:
        if self.matched:
            return (f"sequences match (worst relative difference "
                    f"{self.worst_relative_difference:.3g} at index {self.worst_index})")
        if self.non_finite:
            return (f"non-finite value at index {self.index}: actual {self.actual!r}, "
                    f"expected {self.expected!r}")
        return (f"mismatch at index {self.index}: actual {self.actual:.9g}, expected "
                f"{self.expected:.9g} (absolute {self.absolute_difference:.3g}, relative "
                f"{self.relative_difference:.3g})")


def _flat(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float64).reshape(-1)


def _track_worst(result: Comparison, rel: np.ndarray, stop: int, first_failing: int) -> None:
    """The worst relative difference over the elements the reference's sequential
    loop records before it returns (test_utils.hpp:95-131): every element before
    the stop, plus the stopping element itself when it fails on tolerance (the
    loop records it before the check), not when it is non-finite (returned
    before). Ties keep the first index, as the loop's strict `>` does."""
    scanned = stop + 1 if stop < rel.size and stop == first_failing else stop
    if scanned > 0:
        window = rel[:scanned]
        result.worst_index = int(np.argmax(window))
        result.worst_relative_difference = float(window[result.worst_index])


def compare_close(actual, expected, rtol: float = 1.0e-5, atol: float = 1.0e-6) -> Comparison:
    a, e = _flat(actual), _flat(expected)
    assert a.size == e.size, "compared sequences differ in length"
    result = Comparison()
    finite = np.isfinite(a) & np.isfinite(e)
    same_infinity = np.isinf(a) & np.isinf(e) & (np.signbit(a) == np.signbit(e))
    bad_nonfinite = ~finite & ~same_infinity
    with np.errstate(invalid="ignore"):
        diff = np.where(finite, np.abs(a - e), 0.0)
    mag = np.where(finite, np.abs(e), 0.0)
    rel = np.where(mag > 0, diff / np.where(mag > 0, mag, 1.0), diff)
    failing = finite & (diff > atol + rtol * mag)
    first_nonfinite = int(np.argmax(bad_nonfinite)) if bad_nonfinite.any() else a.size
    first_failing = int(np.argmax(failing)) if failing.any() else a.size
    stop = min(first_nonfinite, first_failing)
    _track_worst(result, rel, stop, first_failing)
    if stop == a.size:
        return result
    result.matched = False
    result.index = stop
    result.actual = float(a[stop])
    result.expected = float(e[stop])
    if stop == first_nonfinite:
        result.non_finite = True
        return result
    result.absolute_difference = float(diff[stop])
    result.relative_difference = float(rel[stop])
    return result


def compare_close_scaled(actual, expected, scale, rtol: float = 1.0e-6,
                         atol: float = 1.0e-6) -> Comparison:
    a, e, s = _flat(actual), _flat(expected), np.abs(_flat(scale))
    assert a.size == e.size == s.size, "compared sequences differ in length"
    result = Comparison()
    bad_nonfinite = ~(np.isfinite(a) & np.isfinite(e) & np.isfinite(s))
    finite = ~bad_nonfinite
    with np.errstate(invalid="ignore"):
        diff = np.where(finite, np.abs(a - e), 0.0)
    mag = np.where(finite, s, 0.0)
    rel = np.where(mag > 0, diff / np.where(mag > 0, mag, 1.0), diff)
    failing = finite & (diff > atol + rtol * mag)
    first_nonfinite = int(np.argmax(bad_nonfinite)) if bad_nonfinite.any() else a.size
    first_failing = int(np.argmax(failing)) if failing.any() else a.size
    stop = min(first_nonfinite, first_failing)
    _track_worst(result, rel, stop, first_failing)
    if stop == a.size:
        return result
    result.matched = False
    result.index = stop
    result.actual = float(a[stop])
    result.expected = float(e[stop])
    if stop == first_nonfinite:
        result.non_finite = True
        return result
    result.absolute_difference = float(diff[stop])
    result.relative_difference = float(rel[stop])
    return result


def require_close(actual, expected, context: str, rtol: float = 1.0e-5,
                  atol: float = 1.0e-6) -> Comparison:
    result = compare_close(actual, expected, rtol, atol)
    if not result:
        raise TestFailure(f"{context}: {result.describe()}")
    return result


def require_close_scaled(actual, expected, scale, context: str, rtol: float = 1.0e-6,
                         atol: float = 1.0e-6) -> Comparison:
    result = compare_close_scaled(actual, expected, scale, rtol, atol)
    if not result:
        raise TestFailure(f"{context}: {result.describe()}")
    return result


def require_exact(actual, expected, context: str) -> None:
    a = np.ascontiguousarray(actual)
    e = np.ascontiguousarray(expected)
    if a.dtype != e.dtype or a.shape != e.shape:
        raise TestFailure(f"{context}: dtype/shape differ ({a.dtype}{a.shape} vs {e.dtype}{e.shape})")
    av = a.reshape(-1).view(np.uint8).reshape(a.size, -1) if a.size else a.reshape(-1)
    ev = e.reshape(-1).view(np.uint8).reshape(e.size, -1) if e.size else e.reshape(-1)
    if a.size and not np.array_equal(av, ev):
        differing = np.nonzero((av != ev).any(axis=1))[0]
        raise TestFailure(f"{context}: values differ at index {int(differing[0])} "
                          f"({differing.size} elements differ)")


def require_max_abs(actual, expected, limit: float, context: str) -> float:
    """Max-abs error bound, finite values only."""
    a, e = _flat(actual), _flat(expected)
    if not (np.isfinite(a).all() and np.isfinite(e).all()):
        raise TestFailure(f"{context}: non-finite values")
    worst = float(np.max(np.abs(a - e))) if a.size else 0.0
    if worst > limit:
        index = int(np.argmax(np.abs(a - e)))
        raise TestFailure(f"{context}: max-abs error {worst:.3g} > {limit:.3g} at index {index}")
    return worst
