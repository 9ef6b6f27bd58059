"""CPU checks of the lift-splat-shoot oracle (oracle/src/lss.c).

Pins, per function:
  * against the reference's own CPU sources compiled as-is (oracle/_ref,
    reference src/lss.c:8-241): bit-identical outputs on the compact case of
    tools/oracle_kernels.py:237-290 and on a small surround rig;
  * against what the mathematics fixes, computed independently in float64
    numpy: the geometry as post_rot^-1 / K^-1 by LAPACK inverses and matrix
    products, the softmax of the depth column, and the pool as a histogram
    scatter (np.add.at) of the lifted features;
  * the cell rule (bf_oracle_lss_ranks) by known answers at cell centres,
    faces and outside points, and against a pooled histogram from the
    reference build;
  * the reference test's rejections (tests/test_lss.c:47-52, 77-82).
"""

import ctypes as C

import numpy as np
import pytest

import oracle
from bfhip import lss_scene

ORACLE = oracle.Oracle("port")


def _desc(d):
    return oracle.lss_desc(d["batches"], d["cameras"], d["depth_bins"], d["height"], d["width"],
                           d["channels"], d["minimum"], d["step"], d["cells"])


def _geometry(o, sc):
    return o.lss_geometry(sc["frustum"], sc["camera_rotation"], sc["camera_translation"],
                          sc["intrinsics"], sc["post_rotation"], sc["post_translation"],
                          sc.get("extra_rotation"), sc.get("extra_translation"))


def _small_rig():
    return lss_scene.rig(seed=3, height=4, width=11, depth_bins=30, channels=8)


def geometry_f64(sc):
    """Frustum -> lidar points in float64 with LAPACK inverses."""
    f = sc["frustum"].astype(np.float64)
    pr = np.linalg.inv(sc["post_rotation"].astype(np.float64))
    comb = sc["camera_rotation"].astype(np.float64) @ np.linalg.inv(
        sc["intrinsics"].astype(np.float64))
    p = f[None, None] - sc["post_translation"].astype(np.float64)[:, :, None, None, None]
    p = np.einsum("bnij,bndhwj->bndhwi", pr, p)
    p = np.concatenate([p[..., :2] * p[..., 2:3], p[..., 2:3]], -1)
    g = np.einsum("bnij,bndhwj->bndhwi", comb, p)
    g += sc["camera_translation"].astype(np.float64)[:, :, None, None, None]
    if sc.get("extra_rotation") is not None:
        g = np.einsum("bij,bndhwj->bndhwi", sc["extra_rotation"].astype(np.float64), g)
    if sc.get("extra_translation") is not None:
        g += sc["extra_translation"].astype(np.float64)[:, None, None, None, None]
    return g


def lift_pool_f64(logits, context, ranks, d):
    """softmax over depth x context, scattered into [B, C*Z, X, Y] by rank."""
    lg = logits.astype(np.float64)
    prob = np.exp(lg - lg.max(2, keepdims=True))
    prob /= prob.sum(2, keepdims=True)
    lifted = prob[:, :, :, None] * context.astype(np.float64)[:, :, None]  # B N D C H W
    b_, n_, dd, c_, h_, w_ = lifted.shape
    X, Y, Z = d["cells"]
    bev = np.zeros((b_, c_, Z * X * Y))
    for b in range(b_):
        r = ranks[b].reshape(-1)
        feats = lifted[b].transpose(0, 1, 3, 4, 2).reshape(-1, c_)
        keep = r >= 0
        acc = np.zeros((Z * X * Y, c_))
        np.add.at(acc, r[keep], feats[keep])
        bev[b] = acc.T
    # rank = (z * X + x) * Y + y  ->  [B, C, Z, X, Y] -> [B, C*Z, X, Y]
    return bev.reshape(b_, c_ * Z, X, Y)


@pytest.mark.parametrize("scene", ["compact", "rig"])
def test_oracle_matches_reference_build_bit_exact(scene):
    if not oracle.available("ref_scalar"):
        pytest.skip("reference CPU sources are not present to build oracle/_ref")
    sc = lss_scene.compact(0) if scene == "compact" else _small_rig()
    d = _desc(sc["desc"])
    with oracle.scalar_env():
        port, ref = oracle.Oracle("port_scalar"), oracle.Oracle("ref_scalar")
        g_port, g_ref = _geometry(port, sc), _geometry(ref, sc)
        assert np.array_equal(g_port.view(np.uint32), g_ref.view(np.uint32))
        lifted = port.lss_lift(sc["depth_logits"], sc["context"], d)
        assert np.array_equal(lifted, ref.lss_lift(sc["depth_logits"], sc["context"], d))
        bev = port.lss_bev_pool(lifted, g_port, d)
        assert np.array_equal(bev, ref.lss_bev_pool(lifted, g_ref, d))
        fused = port.lss_lift_pool(sc["depth_logits"], sc["context"], g_port, d)
        assert np.array_equal(fused, ref.lss_lift_pool(sc["depth_logits"], sc["context"], g_ref,
                                                       d))


@pytest.mark.parametrize("scene", ["compact", "rig"])
def test_geometry_against_float64_algebra(scene):
    sc = lss_scene.compact(0) if scene == "compact" else _small_rig()
    g = _geometry(ORACLE, sc)
    ref = geometry_f64(sc)
    scale = np.abs(ref).max()
    # float32 evaluation of a few dozen operations: relative error ~1e-6 of
    # the coordinate scale.
    assert np.abs(g - ref).max() <= 2e-6 * scale, np.abs(g - ref).max() / scale


@pytest.mark.parametrize("scene", ["compact", "rig"])
def test_lift_and_pool_against_float64_scatter(scene):
    sc = lss_scene.compact(1) if scene == "compact" else _small_rig()
    dd = sc["desc"]
    d = _desc(dd)
    g = _geometry(ORACLE, sc)
    ranks = ORACLE.lss_ranks(g, d)
    lifted = ORACLE.lss_lift(sc["depth_logits"], sc["context"], d)
    lg = sc["depth_logits"].astype(np.float64)
    prob = np.exp(lg - lg.max(2, keepdims=True))
    prob /= prob.sum(2, keepdims=True)
    want = prob[..., None] * sc["context"].astype(np.float64).transpose(0, 1, 3, 4, 2)[:, :,
                                                                                       None]
    assert np.abs(lifted - want).max() <= 1e-6 * np.abs(want).max()
    ref = lift_pool_f64(sc["depth_logits"], sc["context"], ranks, dd)
    assert ranks.max() >= 0 and (ranks >= 0).sum() > 0.2 * ranks.size
    for got in (ORACLE.lss_bev_pool(lifted, g, d),
                ORACLE.lss_lift_pool(sc["depth_logits"], sc["context"], g, d)):
        assert got.shape == ref.shape
        assert np.abs(got - ref).max() <= 1e-5 * max(np.abs(ref).max(), 1e-30)


def test_cell_rule_known_answers():
    dd = dict(batches=1, cameras=1, depth_bins=1, height=1, width=10, channels=1,
              minimum=(-6.0, -6.0, -3.0), step=(2.0, 2.0, 2.0), cells=(6, 6, 4))
    d = _desc(dd)
    pts = np.array([
        [-5.0, -5.0, -2.0],      # centre of cell (0, 0, 0)
        [5.0, -5.0, -2.0],       # x = 5 -> (5, 0, 0)
        [-5.0, 5.0, 4.9],        # y = 5, z = 3
        [-6.0, -6.0, -3.0],      # the grid's minimum corner is inside
        [6.0, 0.0, 0.0],         # x at the far face is outside
        [-6.5, 0.0, 0.0],        # t = -0.25 truncates to 0: inside
        [-8.0, 0.0, 0.0],        # t = -1 -> -1: outside
        [np.nan, 0.0, 0.0],
        [np.inf, 0.0, 0.0],
        [1.0, 1.0, 5.0],         # z = 4 -> outside
    ], np.float32).reshape(1, 1, 1, 1, 10, 3)
    X, Y = 6, 6
    want = [0, (0 * X + 5) * Y + 0, (3 * X + 0) * Y + 5, 0, -1, (1 * X + 0) * Y + 3, -1, -1, -1,
            -1]
    got = ORACLE.lss_ranks(pts, d).ravel().tolist()
    assert got == want


def test_ranks_match_reference_pooled_histogram():
    """With every lifted value 1 and one channel, the reference's pool counts
    the samples per cell; the oracle ranks must give the same histogram."""
    if not oracle.available("ref_scalar"):
        pytest.skip("reference CPU sources are not present to build oracle/_ref")
    sc = _small_rig()
    dd = dict(sc["desc"], channels=1)
    d = _desc(dd)
    g = _geometry(ORACLE, sc)
    ranks = ORACLE.lss_ranks(g, d)
    ones = np.ones(ranks.shape + (1,), np.float32)
    with oracle.scalar_env():
        hist = oracle.Oracle("ref_scalar").lss_bev_pool(ones, g, d).ravel()
    want = np.bincount(ranks[ranks >= 0], minlength=hist.size).astype(np.float32)
    assert np.array_equal(hist, want)


def test_rejections_of_reference_test():
    singular = np.zeros((1, 1, 3, 3), np.float32)
    vec = np.zeros((1, 1, 3), np.float32)
    with pytest.raises(oracle.OracleError):
        ORACLE.lss_geometry(np.zeros((1, 1, 1, 3), np.float32), singular, vec, singular,
                            singular, vec)
    tiny = _desc(dict(batches=1, cameras=1, depth_bins=4, height=1, width=1, channels=1,
                      minimum=(0, 0, 0), step=(1, 1, 1), cells=(1, 1, 1)))
    logits = np.array([0, 0, np.inf, 0], np.float32).reshape(1, 1, 4, 1, 1)
    with pytest.raises(oracle.OracleError):
        ORACLE.lss_lift_pool(logits, np.ones((1, 1, 1, 1, 1), np.float32),
                             np.zeros((1, 1, 4, 1, 1, 3), np.float32), tiny)
    bad = _desc(dict(batches=1, cameras=1, depth_bins=4, height=1, width=1, channels=1,
                     minimum=(0, 0, 0), step=(1, 0, 1), cells=(1, 1, 1)))
    with pytest.raises(oracle.OracleError):
        ORACLE.lss_ranks(np.zeros((1, 1, 4, 1, 1, 3), np.float32), bad)


def test_production_scene_lands_where_the_benchmark_says():
    """The production inputs place sample (cam, d, y, x) in cell
    ((4x + d + 13 cam) % 360, (9y + 3d + 17 cam) % 360) and every frustum
    point (through identity calibration) in ((4x + d) % 360, (9y + 3d) % 360)."""
    sc = lss_scene.production()
    dd = sc["desc"]
    d = _desc(dd)
    ranks = ORACLE.lss_ranks(sc["geometry"], d).reshape(6, 118, 32, 88)
    cam, dep, y, x = np.meshgrid(np.arange(6), np.arange(118), np.arange(32), np.arange(88),
                                 indexing="ij")
    want = ((4 * x + dep + 13 * cam) % 360) * 360 + (9 * y + 3 * dep + 17 * cam) % 360
    assert np.array_equal(ranks, want)
    g = _geometry(ORACLE, sc)
    franks = ORACLE.lss_ranks(g, d).reshape(6, 118, 32, 88)
    assert np.array_equal(franks, ((4 * x + dep) % 360) * 360 + (9 * y + 3 * dep) % 360)
