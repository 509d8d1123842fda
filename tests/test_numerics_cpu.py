"""The comparators every parity test judges through, checked themselves
(reference tests/numerics_test.cu:23-202).

A comparator that wrongly accepted a bad value would turn every parity test
green, so each case below states one property the reference's comparators have
(test_utils.hpp:88-227) and checks it on hand-made values. The cases take the
comparator functions as an argument; `test_planted_comparator_mistakes_are_caught`
runs them against deliberately broken comparators (NaN accepted, the relative
term dropped, the index off by one, ...) and requires that each one turns at
least one case red.
"""

from __future__ import annotations

import types

import numpy as np
import pytest

import numerics
from numerics import Comparison, TestFailure

F32 = np.float32
INF = F32(np.inf)
NAN = F32(np.nan)


def _one(value) -> np.ndarray:
    return np.array([value], dtype=np.float32)


def require(condition: bool, message: str) -> None:
    if not condition:
        raise TestFailure(message)


# -- the cases of numerics_test.cu, one function each -------------------------------------

def case_identical_sequences_match(m) -> None:  # numerics_test.cu:23-28
    values = np.array([0.0, 1.0, -2.5, 1.0e6, 1.0e-6], dtype=np.float32)
    result = m.compare_close(values, values)
    require(bool(result), "identical sequences did not compare equal")
    require(result.worst_relative_difference == 0.0, "identical sequences reported a difference")


def case_single_corrupted_element_is_caught(m) -> None:  # :30-40
    expected = np.ones(64, dtype=np.float32)
    actual = expected.copy()
    actual[37] = 1.5
    result = m.compare_close(actual, expected)
    require(not result, "a corrupted element was accepted")
    require(result.index == 37, "the reported mismatch index is wrong")
    require(result.actual == 1.5 and result.expected == 1.0,
            "the reported values do not name the mismatch")


def case_relative_tolerance_scales_with_magnitude(m) -> None:  # :42-65
    small_expected, large_expected = F32(1.0e-3), F32(1.0e6)
    small_actual = F32(small_expected * F32(1.000001))
    large_actual = F32(large_expected * F32(1.000001))
    require(bool(m.compare_close(_one(small_actual), _one(small_expected), 1.0e-5, 0.0)),
            "a 1e-6 relative error was rejected at small magnitude")
    require(bool(m.compare_close(_one(large_actual), _one(large_expected), 1.0e-5, 0.0)),
            "a 1e-6 relative error was rejected at large magnitude")
    # An absolute difference of 1 is negligible against 1e6 but total against 1e-3.
    shifted_large = F32(large_expected + F32(1.0))
    shifted_small = F32(small_expected + F32(1.0))
    require(bool(m.compare_close(_one(shifted_large), _one(large_expected), 1.0e-5, 0.0)),
            "a negligible error at large magnitude was rejected")
    require(not m.compare_close(_one(shifted_small), _one(small_expected), 1.0e-5, 0.0),
            "a total error at small magnitude was accepted")


def case_absolute_tolerance_covers_zero(m) -> None:  # :67-77
    expected, actual = _one(0.0), _one(1.0e-9)
    require(not m.compare_close(actual, expected, 1.0e-5, 0.0),
            "a difference from zero was accepted with no absolute tolerance")
    require(bool(m.compare_close(actual, expected, 1.0e-5, 1.0e-6)),
            "rounding noise around zero was rejected")


def case_non_finite_values_never_match(m) -> None:  # :79-102
    result = m.compare_close(_one(NAN), _one(NAN))
    require(not result, "NaN compared equal to itself")
    require(result.non_finite, "a NaN mismatch was not reported as non-finite")
    require(not m.compare_close(_one(NAN), _one(1.0)), "NaN compared equal to a finite value")
    require(not m.compare_close(_one(1.0), _one(NAN)), "a finite value compared equal to NaN")
    require(bool(m.compare_close(_one(INF), _one(INF))), "matching infinities were rejected")
    require(not m.compare_close(_one(INF), _one(-INF)),
            "infinities of opposite sign compared equal")
    require(not m.compare_close(_one(INF), _one(1.0e30)),
            "an infinity compared equal to a finite value")


def case_worst_difference_is_tracked_on_success(m) -> None:  # :104-114
    expected = np.full(16, 4.0, dtype=np.float32)
    actual = expected.copy()
    actual[9] = F32(4.0) * (F32(1.0) + F32(1.0e-6))
    result = m.compare_close(actual, expected, 1.0e-5, 0.0)
    require(bool(result), "a within-tolerance difference was rejected")
    require(result.worst_index == 9, "the worst difference was attributed to the wrong index")
    require(result.worst_relative_difference > 0.0,
            "a real difference was reported as no difference")


def case_require_close_reports_context(m) -> None:  # :116-131
    expected = np.ones(8, dtype=np.float32)
    actual = expected.copy()
    actual[3] = 2.0
    seen = False
    try:
        m.require_close(actual, expected, "sample comparison")
    except TestFailure as error:
        seen = "sample comparison" in str(error) and "index 3" in str(error)
    require(seen, "require_close did not report the failing context and index")


def case_require_exact_rejects_near_but_unequal(m) -> None:  # :133-146
    expected = _one(1.0)
    actual = np.nextafter(expected, F32(2.0))
    seen = False
    try:
        m.require_exact(actual, expected, "bitwise comparison")
    except TestFailure:
        seen = True
    require(seen, "require_exact accepted values one ULP apart")
    m.require_exact(expected, expected, "identical values")


def case_scaled_comparison_survives_cancellation(m) -> None:  # :148-163
    expected, actual, term_scale = _one(1.0e-4), _one(1.1e-4), _one(1.0e3)
    require(not m.compare_close(actual, expected, 1.0e-5, 0.0),
            "result-relative comparison accepted a 10% error")
    require(bool(m.compare_close_scaled(actual, expected, term_scale, 1.0e-6, 0.0)),
            "term-relative comparison rejected an error far below one ULP of the terms")


def case_scaled_comparison_still_catches_real_errors(m) -> None:  # :165-180
    expected, actual, term_scale = _one(100.0), _one(110.0), _one(200.0)
    result = m.compare_close_scaled(actual, expected, term_scale, 1.0e-6, 0.0)
    require(not result, "term-relative comparison accepted a 5% error against the terms")
    require(result.index == 0, "the reported mismatch index is wrong")
    require(not m.compare_close_scaled(expected, expected, _one(NAN)),
            "a non-finite scale was accepted")


CASES = [
    case_identical_sequences_match,
    case_single_corrupted_element_is_caught,
    case_relative_tolerance_scales_with_magnitude,
    case_absolute_tolerance_covers_zero,
    case_non_finite_values_never_match,
    case_worst_difference_is_tracked_on_success,
    case_require_close_reports_context,
    case_require_exact_rejects_near_but_unequal,
    case_scaled_comparison_survives_cancellation,
    case_scaled_comparison_still_catches_real_errors,
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: c.__name__[len("case_"):])
def test_comparator_case(case) -> None:
    case(numerics)


# -- cases beyond numerics_test: the array comparator's stopping rule ---------------------

def test_first_of_several_mismatches_is_reported() -> None:
    """The reference's loop stops at the first failing element, whichever kind."""
    expected = np.ones(10, dtype=np.float32)
    actual = expected.copy()
    actual[6], actual[4] = 3.0, NAN
    result = numerics.compare_close(actual, expected)
    assert not result and result.index == 4 and result.non_finite
    actual[4] = 1.0
    result = numerics.compare_close(actual, expected)
    assert not result and result.index == 6 and not result.non_finite
    assert result.absolute_difference == 2.0 and result.relative_difference == 2.0


def test_worst_includes_the_failing_element() -> None:
    """The loop records an element's relative difference before it checks the
    tolerance (test_utils.hpp:115-127), so a failure is also the worst seen."""
    expected = np.ones(5, dtype=np.float32)
    actual = expected.copy()
    actual[1] = F32(1.0) + F32(2.0e-6)
    actual[3] = 5.0
    result = numerics.compare_close(actual, expected)
    assert not result and result.index == 3
    assert result.worst_index == 3 and result.worst_relative_difference == 4.0
    # A non-finite stop is returned before it is recorded.
    actual[3] = NAN
    result = numerics.compare_close(actual, expected)
    assert result.non_finite and result.worst_index == 1


def test_require_exact_distinguishes_signed_zero_and_nan_payloads() -> None:
    """Bitwise means bitwise: -0 is not +0, and two NaN payloads differ."""
    with pytest.raises(TestFailure):
        numerics.require_exact(_one(-0.0), _one(0.0), "signed zero")
    quiet = np.array([0x7FC00000], dtype=np.uint32).view(np.float32)
    other = np.array([0x7FC00001], dtype=np.uint32).view(np.float32)
    with pytest.raises(TestFailure):
        numerics.require_exact(quiet, other, "NaN payload")
    numerics.require_exact(quiet, quiet.copy(), "same NaN")


def test_require_max_abs_bounds_and_rejects_nan() -> None:
    expected = np.zeros(4, dtype=np.float32)
    assert numerics.require_max_abs(expected + F32(1.0e-6), expected, 1.0e-5, "within") > 0
    with pytest.raises(TestFailure):
        numerics.require_max_abs(expected + F32(2.0e-5), expected, 1.0e-5, "beyond")
    with pytest.raises(TestFailure):
        numerics.require_max_abs(np.array([0, NAN, 0, 0], np.float32), expected, 1.0, "nan")


# -- the generator half (numerics_test.cu:182-202) ----------------------------------------

def test_generator_is_reproducible(oracle) -> None:
    first = oracle.generator(1234).normal(256)
    second = oracle.generator(1234).normal(256)
    different = oracle.generator(5678).normal(256)
    numerics.require_exact(first, second, "the same seed produced different data")
    assert not np.array_equal(first, different), "different seeds produced identical data"


def test_generator_respects_bounds(oracle) -> None:
    values = oracle.generator(99).uniform(4096, -2.0, 3.0)
    assert np.isfinite(values).all(), "a uniform sample was not finite"
    assert ((values >= -2.0) & (values <= 3.0)).all(), "a uniform sample fell outside its bounds"


# -- planted mistakes: each broken comparator must fail at least one case ------------------

def _mutant(**overrides) -> types.SimpleNamespace:
    functions = dict(compare_close=numerics.compare_close,
                     compare_close_scaled=numerics.compare_close_scaled,
                     require_close=numerics.require_close,
                     require_exact=numerics.require_exact)
    functions.update(overrides)
    return types.SimpleNamespace(**functions)


def _nan_accepted(actual, expected, rtol=1.0e-5, atol=1.0e-6) -> Comparison:
    a = np.asarray(actual, np.float64).reshape(-1)
    e = np.asarray(expected, np.float64).reshape(-1)
    both = np.isnan(a) | np.isnan(e)
    return numerics.compare_close(np.where(both, 0.0, a), np.where(both, 0.0, e), rtol, atol)


def _relative_term_dropped(actual, expected, rtol=1.0e-5, atol=1.0e-6) -> Comparison:
    return numerics.compare_close(actual, expected, 0.0, atol)


def _absolute_term_dropped(actual, expected, rtol=1.0e-5, atol=1.0e-6) -> Comparison:
    return numerics.compare_close(actual, expected, rtol, 0.0)


def _index_off_by_one(actual, expected, rtol=1.0e-5, atol=1.0e-6) -> Comparison:
    result = numerics.compare_close(actual, expected, rtol, atol)
    if not result:
        result.index += 1
    return result


def _worst_untracked(actual, expected, rtol=1.0e-5, atol=1.0e-6) -> Comparison:
    result = numerics.compare_close(actual, expected, rtol, atol)
    result.worst_relative_difference, result.worst_index = 0.0, 0
    return result


def _infinities_any_sign(actual, expected, rtol=1.0e-5, atol=1.0e-6) -> Comparison:
    a = np.asarray(actual, np.float64).reshape(-1)
    e = np.asarray(expected, np.float64).reshape(-1)
    return numerics.compare_close(np.abs(a), np.abs(e), rtol, atol)


def _scale_ignored(actual, expected, scale, rtol=1.0e-6, atol=1.0e-6) -> Comparison:
    return numerics.compare_close(actual, expected, rtol, atol)


def _scale_nan_accepted(actual, expected, scale, rtol=1.0e-6, atol=1.0e-6) -> Comparison:
    s = np.asarray(scale, np.float64)
    return numerics.compare_close_scaled(actual, expected, np.where(np.isfinite(s), s, 0.0),
                                         rtol, atol)


def _exact_within_tolerance(actual, expected, context) -> None:
    if not np.allclose(actual, expected, rtol=1.0e-6, atol=0.0, equal_nan=True):
        raise TestFailure(f"{context}: values differ")


def _require_close_without_context(actual, expected, context, rtol=1.0e-5, atol=1.0e-6):
    result = numerics.compare_close(actual, expected, rtol, atol)
    if not result:
        raise TestFailure("comparison failed")
    return result


MUTANTS = {
    "nan_accepted": _mutant(compare_close=_nan_accepted),
    "relative_term_dropped": _mutant(compare_close=_relative_term_dropped),
    "absolute_term_dropped": _mutant(compare_close=_absolute_term_dropped),
    "index_off_by_one": _mutant(compare_close=_index_off_by_one),
    "worst_untracked": _mutant(compare_close=_worst_untracked),
    "infinities_any_sign": _mutant(compare_close=_infinities_any_sign),
    "scale_ignored": _mutant(compare_close_scaled=_scale_ignored),
    "scale_nan_accepted": _mutant(compare_close_scaled=_scale_nan_accepted),
    "exact_within_tolerance": _mutant(require_exact=_exact_within_tolerance),
    "require_close_without_context": _mutant(require_close=_require_close_without_context),
}


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_comparator_mistakes_are_caught(name) -> None:
    broken = MUTANTS[name]
    failures = []
    for case in CASES:
        try:
            case(broken)
        except TestFailure:
            failures.append(case.__name__)
    assert failures, f"the planted comparator mistake '{name}' passed every case"
