"""The device GELU (hip_common.h gelu()) against the exact-erf GELU of the
reference (kernels_ref.c:448-452), on the CPU.

The device evaluates x * sigmoid(x * p(x^2)), p a quartic in x^2, with no
clamp.  This restates those float32 steps in numpy (fma rounding aside) and
checks them against scipy's erf over the real line: absolute error <= 1e-5
everywhere, relative error below a quarter of the fp16 half-ulp (2^-12, the
device GELU's output is stored as fp16) wherever |GELU| > 0.01, exact zero at
0, the limits (x for large positive x, 0 for large negative x, the reference
formula's inf / NaN at +-inf), the exponent inside the sigmoid monotone and p
negative up to float32's largest x^2, and the reference's GELU fixture grid
linspace(-8, 8, 65)
(tools/oracle_kernels.py:127-129, read by tests/test_kernels.c:89-98) held to
1e-5.
"""

import numpy as np
from scipy.special import erf

# p(t) = K[0] + K[1] t + ... + K[4] t^4, as hip_common.h gelu() holds them
K = np.array([-2.301823854e+00, -1.055332273e-01, 4.688421031e-04,
              7.499327330e-05, -2.720398243e-06], np.float32)


def gelu_device(x):
    x = np.asarray(x, np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        t = x * x
        p = t * K[4] + K[3]
        for k in K[2::-1]:
            p = t * p + k
        e = np.exp2(x * p)
        return x * (np.float32(1) / (np.float32(1) + e))


def gelu_exact(x):
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1 + erf(x / np.sqrt(2)))


def test_absolute_bound_everywhere():
    x = np.concatenate([np.linspace(-60, 60, 1200001), np.linspace(-1e-3, 1e-3, 2001)])
    err = np.abs(gelu_device(x) - gelu_exact(x.astype(np.float32)))
    assert err.max() <= 1e-5, err.max()


def test_relative_error_below_fp16_half_ulp():
    x = np.linspace(-12, 12, 480001).astype(np.float32)
    ref = gelu_exact(x)
    big = np.abs(ref) > 1e-2
    rel = np.abs(gelu_device(x)[big] - ref[big]) / np.abs(ref[big])
    assert rel.max() < 2.0 ** -14, rel.max()


def test_special_values_and_limits():
    assert gelu_device(np.array([0.0]))[0] == 0.0
    big = np.array([10.0, 25.0, 1e4, 3e38], np.float32)
    np.testing.assert_allclose(gelu_device(big), big, rtol=1e-7)
    assert np.all(np.abs(gelu_device(-big)) <= 1e-7 * big)
    # 0.5 x (1 + erf(x / sqrt 2)) at +-inf: inf, and -inf * 0 = NaN
    y = gelu_device(np.array([np.inf, -np.inf, np.nan], np.float32))
    assert y[0] == np.inf and np.isnan(y[1]) and np.isnan(y[2])


def test_sigmoid_exponent_monotone_and_negative():
    """x * p(x^2) must fall monotonically (else the sigmoid would turn back),
    and p must stay negative for every float32 x^2 (then 2^(x p) only
    saturates: to 0 for large positive x, to +inf for large negative x)."""
    x = np.linspace(0, 100, 1000001)
    u = x * np.polyval(K[::-1].astype(np.float64), x * x)
    assert np.all(np.diff(u) < 0)
    assert u[np.searchsorted(x, 6.0)] < -39
    t = np.concatenate([np.linspace(0, 1e4, 1000001), np.logspace(4, 38.5, 10001)]).astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        p = t * K[4] + K[3]
        for k in K[2::-1]:
            p = t * p + k
    assert not np.isnan(p).any() and p.max() < 0


def test_reference_fixture_grid():
    x = np.linspace(-8, 8, 65)  # tools/oracle_kernels.py GELU fixture grid
    assert np.max(np.abs(gelu_device(x) - gelu_exact(x))) <= 1e-5
