"""Fits the polynomial of the branch-free erfc behind the GELU kernels.

The device GELU (device_common.hpp, gelu()) evaluates
    erfc(z) = t * exp(-z^2 + P(t)),   t = 1 / (1 + z / 2),   z >= 0,
the functional form of the Chebyshev erfc approximation in Press et al.,
Numerical Recipes (section 6.2, "erfcc"). An error dP in P is a relative error
exp(dP) - 1 of erfc, so fitting P uniformly gives erfc to a uniform relative
accuracy. This script fits P, a degree-7 polynomial in t, by Chebyshev
interpolation (near-minimax) in float64 over z in [0, 10]
(t in [1/6, 1]) and prints the largest error of the fit. Beyond z = 10,
erfc(z) < 2e-45 is below float32 anyway.

The device evaluates in base 2, erfc(z) / 2 = t exp2(-w^2 + Q(t)) with
w = z sqrt(log2 e) and Q = P log2 e - 1 (the -1 is the factor 1/2), so the
script prints Q's coefficients, lowest power first, and the two scale
constants of w and t. Run: python3 gelu_fit.py (needs numpy and scipy; the
CPU tests import it to check the header against it; not used by the build).
"""

import numpy as np
from scipy.special import log_ndtr

Z_MAX = 10.0
DEGREE = 7


def target(t):
    """ln(erfc(z)) + z^2 - ln(t) at z = 2 (1 / t - 1)."""
    z = 2.0 * (1.0 / t - 1.0)
    log_erfc = np.log(2.0) + log_ndtr(-z * np.sqrt(2.0))  # erfc(z) = 2 Phi(-z sqrt 2)
    return log_erfc + z * z - np.log(t)


def fit(degree=DEGREE, z_max=Z_MAX):
    t_lo = 1.0 / (1.0 + z_max / 2.0)
    nodes = np.cos(np.pi * (np.arange(4000) + 0.5) / 4000)
    t = t_lo + (1.0 - t_lo) * (nodes + 1.0) / 2.0
    cheb = np.polynomial.chebyshev.Chebyshev.fit(t, target(t), degree, domain=[t_lo, 1.0])
    poly = cheb.convert(kind=np.polynomial.Polynomial)
    grid = np.linspace(t_lo, 1.0, 200001)
    return poly.coef, float(np.abs(poly(grid) - target(grid)).max())


LOG2E = 1.0 / np.log(2.0)
W_SCALE = np.sqrt(LOG2E / 2.0)     # w = |x| W_SCALE = (|x| / sqrt 2) sqrt(log2 e)
T_SCALE = 0.5 / np.sqrt(LOG2E)     # 1 + z / 2 = 1 + w T_SCALE


def folded(degree=DEGREE, z_max=Z_MAX):
    """Q = P log2(e) - 1, lowest power first, and the fit's largest error."""
    coefficients, error = fit(degree, z_max)
    q = coefficients * LOG2E
    q[0] -= 1.0
    return q, error


if __name__ == "__main__":
    q, error = folded()
    print(f"max |dP| = {error:.3e} over z in [0, {Z_MAX}]")
    print(f"w scale = {W_SCALE:.17g}, t scale = {T_SCALE:.17g}")
    for power, c in enumerate(q):
        print(f"q{power} = {c:.9e}")
