"""The GELU the kernels compute (device_common.hpp, gelu()), evaluated on the
CPU step by step in float32, against the erf GELU in float64.

The device form is erfc(z) = t * exp(-z^2 + P(t)), t = 1 / (1 + z / 2),
z = |x| / sqrt(2), evaluated in base 2 as erfc(z) / 2 = t exp2(-w^2 + Q(t))
with w = z sqrt(log2 e) and Q = P log2 e - 1. The degree-7 polynomial Q and
the two scale constants are read from the header here, so a changed
coefficient or a changed step is caught without a GPU. The GPU tests hold the
kernels themselves to the oracle (std::erf).
"""

from __future__ import annotations

import os
import re
from pathlib import Path

import numpy as np
import pytest

from conftest import ROOT

scipy_special = pytest.importorskip("scipy.special")

HEADER = os.path.join(ROOT, "cu-vit_amd", "csrc", "kernels", "device_common.hpp")
F32 = np.float32


def gelu_body():
    text = Path(HEADER).read_text()
    body = text[text.index("__device__ __forceinline__ float gelu(float x)"):]
    return body[:body.index("return")]


def coefficients():
    """Q's coefficients from the header, highest power first (Horner order)."""
    body = gelu_body()
    first = re.search(r"float q = ([-+0-9.eE]+)F;", body).group(1)
    rest = re.findall(r"q = fmaf\(q, t, ([-+0-9.eE]+)F\);", body)
    return [F32(first)] + [F32(c) for c in rest]


def scales():
    """The constants of w = |x| * W and of 1 + w * T, from the header."""
    body = gelu_body()
    w = re.search(r"fabsf\(x\) \* ([-+0-9.eE]+)F;", body).group(1)
    t = re.search(r"fmaf\(w, ([-+0-9.eE]+)F, 1\.0F\)", body).group(1)
    return F32(w), F32(t)


def fma(a, b, c):
    # float32 fused multiply-add: the product of two float32 values is exact in
    # float64, so one rounding of the sum to float32 remains
    return (a.astype(np.float64) * b.astype(np.float64) + c).astype(F32)


def device_gelu(x):
    x = x.astype(F32)
    w_scale, t_scale = scales()
    w = (np.abs(x) * w_scale).astype(F32)
    t = (1.0 / fma(w, np.full_like(w, t_scale), np.float64(1.0)).astype(np.float64)).astype(F32)
    c = coefficients()
    q = np.full_like(t, c[0])
    for coefficient in c[1:]:
        q = fma(q, t, np.float64(coefficient))
    exponent = fma(-w, w, q.astype(np.float64))
    e = np.exp2(exponent.astype(np.float64)).astype(F32)
    half = (t * e).astype(F32)
    return (x * np.where(x < 0, half, fma(-t, e, np.float64(1.0)))).astype(F32)


def exact_gelu(x):
    x = x.astype(np.float64)
    return 0.5 * x * scipy_special.erfc(-x / np.sqrt(2.0))


def test_header_has_the_degree_seven_polynomial():
    assert len(coefficients()) == 8


def test_dense_grid_against_float64():
    x = np.linspace(-12.0, 12.0, 400001).astype(F32)
    error = np.abs(device_gelu(x).astype(np.float64) - exact_gelu(x))
    assert error.max() < 5.0e-7
    # the reference test's tolerance for GELU (elementwise_test.cu:48-49)
    assert np.all(error <= 1.0e-6 + 1.0e-5 * np.abs(exact_gelu(x)))


def test_landmarks_of_the_reference_test():
    """elementwise_test.cu:38-42's landmark inputs."""
    x = np.array([-30, -8, -2.7, -2, -1, -0.5, 0, 0.5, 1, 2, 2.7, 8, 30], F32)
    got = device_gelu(x).astype(np.float64)
    expected = exact_gelu(x)
    assert np.all(np.abs(got - expected) <= 1.0e-6 + 1.0e-5 * np.abs(expected))
    assert got[6] == 0.0 and got[-1] == 30.0


def test_negative_tail_keeps_relative_accuracy():
    """Where 1 + erf cancels (the textbook formula loses every digit by x = -6),
    the erfc form stays relatively accurate; what remains is the rounding of
    w and of the exponent -w^2 + Q(t) before exp2, about 1e-7 relative per
    unit of z^2."""
    x = np.linspace(-9.0, -3.0, 20001).astype(F32)
    expected = exact_gelu(x)
    relative = np.abs(device_gelu(x).astype(np.float64) - expected) / np.abs(expected)
    assert relative.max() < 1.0e-5


def test_fit_script_reproduces_the_error_bound():
    import importlib.util

    spec = importlib.util.spec_from_file_location(
        "gelu_fit", os.path.join(ROOT, "cu-vit_amd", "csrc", "kernels", "gelu_fit.py"))
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    fitted, error = module.folded()
    assert error < 7.5e-7
    header = np.array(coefficients()[::-1], F32)  # lowest power first
    assert np.array_equal(header, fitted.astype(F32))
    assert scales() == (F32(module.W_SCALE), F32(module.T_SCALE))


def test_bf16_results_round_like_the_exact_gelu():
    """Rounded to bf16, as the bf16 GEMM epilogue stores it, the device form
    lands on the correctly rounded GELU for all but a few in 1e4 inputs."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(1 << 20) * 2.0).astype(F32)

    def bf16(v):
        u = v.astype(F32).view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)

    flips = np.count_nonzero(bf16(device_gelu(x)) != bf16(exact_gelu(x).astype(F32)))
    assert flips / x.size < 2.0e-4


def test_special_values():
    """+inf stays +inf, NaN stays NaN; -inf gives NaN as 0.5 x (1 + erf) does."""
    with np.errstate(invalid="ignore"):  # -inf * 0 and NaN, as on the device
        got = device_gelu(np.array([np.inf, -np.inf, np.nan], F32))
    assert got[0] == np.inf and np.isnan(got[1]) and np.isnan(got[2])
