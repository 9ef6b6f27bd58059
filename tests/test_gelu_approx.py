"""The device GELU's erf is Abramowitz & Stegun formula 7.1.26 (CPU check).

Restates the polynomial in float64 numpy and checks it against scipy's erf
over the whole real line: the published bound |error| <= 1.5e-7 holds, so the
GELU feeding bf16 storage differs from the exact-erf reference
(kernels_ref.c:448-452) far below the north-star tolerance.
"""

import numpy as np
from scipy.special import erf

P = 0.3275911
A = (0.254829592, -0.284496736, 1.421413741, -1.453152027, 1.061405429)


def erf_as(x):
    z = np.abs(x)
    t = 1.0 / (1.0 + P * z)
    poly = t * (A[0] + t * (A[1] + t * (A[2] + t * (A[3] + t * A[4]))))
    return np.sign(x) * (1.0 - poly * np.exp(-z * z))


def test_erf_bound():
    x = np.linspace(-9, 9, 200001)
    assert np.max(np.abs(erf_as(x) - erf(x))) <= 1.5e-7


def test_gelu_error_relative_to_bf16():
    x = np.linspace(-8, 8, 65)  # the reference's GELU fixture grid
    exact = 0.5 * x * (1 + erf(x / np.sqrt(2)))
    approx = 0.5 * x * (1 + erf_as(x / np.sqrt(2)))
    assert np.max(np.abs(approx - exact)) <= 8 * 1.5e-7 * 0.5 + 1e-12
    assert erf_as(np.array([0.0]))[0] == 0.0
