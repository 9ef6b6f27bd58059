"""The device GELU (hip_common.h gelu()) against the exact-erf GELU of the
reference (kernels_ref.c:448-452), on the CPU.

The device evaluates x * sigmoid(x * (a + b x^2 + c x^4)) with x clamped to
[-10, 10] inside the sigmoid.  This restates those float32 steps in numpy
(fma rounding aside) and checks them against scipy's erf over the real line:
absolute error <= 3e-5 everywhere, relative error below the bf16 half-ulp
wherever |GELU| > 0.01, exact zero at 0, odd-symmetric limits (x for large
positive x, 0 for large negative x), and the reference's GELU fixture grid
linspace(-8, 8, 65) (tools/oracle_kernels.py:127-129, read by
tests/test_kernels.c:89-98) held to 3e-5.
"""

import numpy as np
from scipy.special import erf

K = np.array([-2.301121339e+00, -1.067757240e-01, 1.014263055e-03], np.float32)


def gelu_device(x):
    x = np.asarray(x, np.float32)
    xc = np.clip(x, np.float32(-10), np.float32(10))
    t = xc * xc
    p = t * K[2] + K[1]
    p = t * p + K[0]
    with np.errstate(over="ignore"):
        e = np.exp2(xc * p)
    return x * (np.float32(1) / (np.float32(1) + e))


def gelu_exact(x):
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1 + erf(x / np.sqrt(2)))


def test_absolute_bound_everywhere():
    x = np.concatenate([np.linspace(-60, 60, 1200001), np.linspace(-1e-3, 1e-3, 2001)])
    err = np.abs(gelu_device(x) - gelu_exact(x.astype(np.float32)))
    assert err.max() <= 3e-5, err.max()


def test_relative_error_below_bf16_half_ulp():
    x = np.linspace(-12, 12, 480001).astype(np.float32)
    ref = gelu_exact(x)
    big = np.abs(ref) > 1e-2
    rel = np.abs(gelu_device(x)[big] - ref[big]) / np.abs(ref[big])
    assert rel.max() < 2.0 ** -9


def test_special_values_and_limits():
    assert gelu_device(np.array([0.0]))[0] == 0.0
    big = np.array([10.0, 25.0, 1e4], np.float32)
    np.testing.assert_allclose(gelu_device(big), big, rtol=1e-7)
    assert np.all(np.abs(gelu_device(-big)) <= 1e-7 * big)


def test_reference_fixture_grid():
    x = np.linspace(-8, 8, 65)  # tools/oracle_kernels.py GELU fixture grid
    assert np.max(np.abs(gelu_device(x) - gelu_exact(x))) <= 3e-5
