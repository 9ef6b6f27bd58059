"""Numerical helpers shared by the tests."""

import numpy as np

# Tolerance stated by BASELINE.json north_star for bf16-in / fp32-accumulate
# floating-point outputs against the fp32 CPU oracle.
REL_L2 = 1e-2
MAX_ABS_RMS = 5e-2


def pattern(i):
    """Deterministic fill of the reference GPU op tests (test_cuda_ops.cu:11-13)."""
    i = np.asarray(i, dtype=np.int64)
    return (((i * 37) % 101) - 50).astype(np.float32) / np.float32(37.0)


def bf16_round(x):
    """Round float32 to the nearest bf16 (ties to even), keeping NaN/Inf."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    return np.where(np.isfinite(x), r, x).astype(np.float32)


def errors(actual, expected):
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    rms = np.sqrt(np.mean(e * e)) if e.size else 0.0
    diff = a - e
    rel_l2 = np.linalg.norm(diff) / max(np.linalg.norm(e), 1e-30)
    max_abs = np.max(np.abs(diff)) if e.size else 0.0
    return rel_l2, max_abs, rms


def assert_close(actual, expected, name="", rel_l2=REL_L2, max_abs_rms=MAX_ABS_RMS):
    """relative L2 and max-abs relative to output RMS.

    Non-finite expected values must be matched exactly (NaN by NaN, +-Inf by
    the same infinity); the finite remainder is held to the tolerance.
    """
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    assert a.shape == e.shape, f"{name}: shape {a.shape} != {e.shape}"
    bad_nan = np.isnan(a) != np.isnan(e)
    assert not bad_nan.any(), f"{name}: NaN pattern differs at {np.flatnonzero(bad_nan)[:8]}"
    inf_e = np.isinf(e)
    assert np.array_equal(np.isinf(a), inf_e), f"{name}: Inf pattern differs"
    assert np.array_equal(a[inf_e], e[inf_e]), f"{name}: Inf signs differ"
    fin = np.isfinite(e)
    rl2, mabs, rms = errors(a[fin], e[fin])
    print(f"[parity] {name}: rel_l2={rl2:.3e} max_abs/rms={mabs / max(rms, 1e-30):.3e}")
    assert rl2 <= rel_l2, f"{name}: rel L2 {rl2:.3e} > {rel_l2:.1e}"
    assert mabs <= max_abs_rms * rms, f"{name}: max abs {mabs:.3e} > {max_abs_rms} x rms {rms:.3e}"
    return rl2, mabs / max(rms, 1e-30)


def clustered_sites(seed, n, d, h, w):
    """Unique sparse sites [M,4] (batch 0, z, y, x) in six clusters over a
    d x h x w grid, shuffled, so convolution taps find neighbours."""
    rng = np.random.default_rng(seed)
    centres = rng.integers(0, [d, h, w], size=(6, 3))
    pts = centres[rng.integers(0, 6, n)] + rng.integers(-2, 3, size=(n, 3))
    pts = np.clip(pts, 0, [d - 1, h - 1, w - 1])
    uniq = np.unique(pts, axis=0)
    rng.shuffle(uniq)
    return np.concatenate([np.zeros((len(uniq), 1), np.int32), uniq.astype(np.int32)], 1)
