"""Lift-splat-shoot pooling on the GPU (include/bf_cuda.h) against the CPU oracle.

Follows the reference's tests/test_cuda_lss.cu: ranks bit-exact against the
cell rule (:268-291); the stateless atomic routes and the plan route within
tolerance of the CPU pool (:292-340); the production inputs (:26-104) through
both prepare routes.  Beyond the reference test: the plan route is
bit-identical across repeats, re-prepares and HIP-graph replays; preparing
from calibration gives bit-for-bit the lists of preparing from the oracle's
geometry (the calibration transform follows the oracle's float operation
order); channel counts that take the scalar and multi-pass pool paths; empty,
non-finite and singular-camera inputs.

Tolerance (float32 sums in a different order than the oracle, and expf
within an ulp): per element |gpu - oracle| <= 1e-6 max(M) + 2e-5 M, where
M = the oracle pool of |context| (the sum of the magnitudes of the terms).
The compact case also meets the reference test's own 2e-6 + 8e-6 |ref|.
"""

import numpy as np
import pytest

import bfhip
import oracle
from bfhip import lss_scene

pytestmark = pytest.mark.gpu
ORACLE = oracle.Oracle("port")


def _dev(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def _descs(dd):
    args = (dd["batches"], dd["cameras"], dd["depth_bins"], dd["height"], dd["width"],
            dd["channels"], dd["minimum"], dd["step"], dd["cells"])
    return bfhip.lss_desc(*args), oracle.lss_desc(*args)


def _geometry(sc):
    """The scene's geometry tensor: given, or the oracle's from its calibration."""
    if "geometry" in sc:
        return sc["geometry"]
    return _frustum_geometry(sc)


def _frustum_geometry(sc):
    return ORACLE.lss_geometry(sc["frustum"], sc["camera_rotation"], sc["camera_translation"],
                               sc["intrinsics"], sc["post_rotation"], sc["post_translation"],
                               sc.get("extra_rotation"), sc.get("extra_translation"))


def _check(got, logits, context, geometry, od, name):
    want = ORACLE.lss_lift_pool(logits, context, geometry, od)
    mag = ORACLE.lss_lift_pool(logits, np.abs(context), geometry, od)
    bound = 1e-6 * mag.max() + 2e-5 * mag
    err = np.abs(got.astype(np.float64) - want)
    print(f"[parity] {name}: max_abs={err.max():.3e} max_err/bound={np.max(err / np.maximum(bound, 1e-30)):.3f}")
    assert got.shape == want.shape
    assert np.all(err <= bound), f"{name}: max abs {err.max():.3e}"
    return want


class _Scenes(dict):
    """Scenes built on first use (not at collection)."""
    MAKERS = {
        "compact": lambda: lss_scene.compact(0),
        "rig_small": lambda: lss_scene.rig(seed=1, height=8, width=22, depth_bins=118,
                                           channels=80),
        "production": lss_scene.production,
        "rig": lambda: lss_scene.rig(seed=2),
    }

    def __missing__(self, key):
        self[key] = self.MAKERS[key]()
        return self[key]


SCENES = _Scenes()
NAMES = list(_Scenes.MAKERS)


@pytest.mark.parametrize("name", NAMES)
def test_ranks_bit_exact(name, device):
    sc = SCENES[name]
    bd, od = _descs(sc["desc"])
    g = _geometry(sc)
    ranks = bfhip.lss_geometry_to_ranks(_dev(g, device), bd)
    assert np.array_equal(ranks.cpu().numpy(), ORACLE.lss_ranks(g, od))


def test_ranks_edge_points(device):
    dd = dict(batches=1, cameras=1, depth_bins=1, height=1, width=12, channels=1,
              minimum=(-6.0, -6.0, -3.0), step=(2.0, 2.0, 2.0), cells=(6, 6, 4))
    bd, od = _descs(dd)
    pts = np.array([[-5, -5, -2], [5, -5, -2], [-5, 5, 4.9], [-6, -6, -3], [6, 0, 0],
                    [-6.5, 0, 0], [-8, 0, 0], [np.nan, 0, 0], [np.inf, 0, 0], [1, 1, 5],
                    [-np.inf, 0, 0], [3e9, 0, 0]], np.float32).reshape(1, 1, 1, 1, 12, 3)
    got = bfhip.lss_geometry_to_ranks(_dev(pts, device), bd).cpu().numpy()
    assert np.array_equal(got, ORACLE.lss_ranks(pts, od))
    assert got.ravel().tolist()[:4] == [0, 30, 113, 0]


@pytest.mark.parametrize("name", NAMES)
def test_plan_geometry_route(name, device):
    import torch
    sc = SCENES[name]
    bd, od = _descs(sc["desc"])
    g = _geometry(sc)
    logits, ctx = _dev(sc["depth_logits"], device), _dev(sc["context"], device)
    with bfhip.LssPlan(bd) as plan:
        plan.prepare_geometry(_dev(g, device))
        out = plan.forward(logits, ctx)
        again = plan.forward(logits, ctx)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.array_equal(got, again.cpu().numpy()), "plan forward is not repeatable"
        want = _check(got, sc["depth_logits"], sc["context"], g, od, f"lss plan {name}")
        if name == "compact":
            assert np.all(np.abs(got - want) <= 2e-6 + 8e-6 * np.abs(want))
        # re-preparing from the same geometry rebuilds identical lists
        plan.prepare_geometry(_dev(g, device))
        assert np.array_equal(plan.forward(logits, ctx).cpu().numpy(), got)
        assert plan.resident_bytes() > 0


@pytest.mark.parametrize("name", ["compact", "rig_small", "production", "rig"])
def test_plan_calibration_route_equals_geometry_route(name, device):
    sc = SCENES[name]
    bd, od = _descs(sc["desc"])
    g = _frustum_geometry(sc)
    logits, ctx = _dev(sc["depth_logits"], device), _dev(sc["context"], device)
    cal = [_dev(sc[k], device) for k in lss_scene.CALIBRATION_KEYS]
    with bfhip.LssPlan(bd) as a, bfhip.LssPlan(bd) as b:
        a.prepare_geometry(_dev(g, device))
        b.prepare_calibration(_dev(sc["frustum"], device), *cal)
        ga, gb = a.forward(logits, ctx).cpu().numpy(), b.forward(logits, ctx).cpu().numpy()
    assert np.array_equal(ga, gb)
    _check(gb, sc["depth_logits"], sc["context"], g, od, f"lss calibration {name}")


def test_calibration_without_extra_transform(device):
    sc = dict(SCENES["compact"], extra_rotation=None, extra_translation=None)
    bd, od = _descs(sc["desc"])
    g = _geometry(sc)
    logits, ctx = _dev(sc["depth_logits"], device), _dev(sc["context"], device)
    cal = [_dev(sc[k], device) for k in lss_scene.CALIBRATION_KEYS[:5]]
    with bfhip.LssPlan(bd) as plan:
        plan.prepare_calibration(_dev(sc["frustum"], device), *cal)
        got = plan.forward(logits, ctx).cpu().numpy()
    _check(got, sc["depth_logits"], sc["context"], g, od, "lss calibration, no extra")


def test_singular_camera_contributes_nothing(device):
    sc = dict(SCENES["rig_small"])
    sc["intrinsics"] = sc["intrinsics"].copy()
    sc["intrinsics"][0, 2] = 0.0  # camera 2: singular intrinsics
    bd, od = _descs(sc["desc"])
    g = _frustum_geometry(SCENES["rig_small"]).copy()
    g[0, 2] = np.nan  # the oracle's equivalent: camera 2 lands nowhere
    logits, ctx = _dev(sc["depth_logits"], device), _dev(sc["context"], device)
    cal = [_dev(sc[k], device) for k in lss_scene.CALIBRATION_KEYS]
    with bfhip.LssPlan(bd) as a, bfhip.LssPlan(bd) as b:
        a.prepare_calibration(_dev(sc["frustum"], device), *cal)
        b.prepare_geometry(_dev(g, device))
        ga, gb = a.forward(logits, ctx).cpu().numpy(), b.forward(logits, ctx).cpu().numpy()
    assert np.array_equal(ga, gb)
    _check(ga, sc["depth_logits"], sc["context"], g, od, "lss singular camera")


@pytest.mark.parametrize("channels", [1, 3, 70, 80, 256, 260])
def test_plan_channel_widths_and_ragged_grid(channels, device):
    """Scalar (C % 4 != 0) and float4 lanes, one and several channel passes,
    two batches with different rigs, Z = 2, a cell count not a multiple of 64."""
    a = lss_scene.rig(seed=5, height=6, width=14, depth_bins=40, channels=channels)
    b = lss_scene.rig(seed=6, height=6, width=14, depth_bins=40, channels=channels)
    b["extra_rotation"] = lss_scene._rot_z(-0.4).reshape(1, 3, 3)
    sc = {k: np.concatenate([a[k], b[k]]) for k in
          ("depth_logits", "context", *lss_scene.CALIBRATION_KEYS)}
    sc["frustum"] = a["frustum"]
    sc["desc"] = dict(a["desc"], batches=2, minimum=(-20.0, -16.0, -2.0), step=(0.55, 0.4, 2.5),
                      cells=(71, 83, 2))
    bd, od = _descs(sc["desc"])
    g = _geometry(sc)
    logits, ctx = _dev(sc["depth_logits"], device), _dev(sc["context"], device)
    with bfhip.LssPlan(bd) as plan:
        plan.prepare_geometry(_dev(g, device))
        got = plan.forward(logits, ctx).cpu().numpy()
    _check(got, sc["depth_logits"], sc["context"], g, od, f"lss plan C={channels}")


def _exact_inputs(sc, seed):
    """Logits with 32 equal maxima per pixel (probabilities exactly 1/32, the
    rest exactly 0) and small-integer context: every partial sum is exact in
    float32, so any summation order must reproduce the oracle bit for bit."""
    rng = np.random.default_rng(seed)
    b, n, d, h, w = sc["depth_logits"].shape
    keys = rng.random((b, n, d, h, w))
    on = np.argsort(keys, axis=2) < 32
    logits = np.where(on, 0.0, -200.0).astype(np.float32)
    ctx = rng.integers(-8, 9, size=sc["context"].shape).astype(np.float32)
    return logits, ctx


@pytest.mark.parametrize("channels,cells", [(260, (8, 8, 1)), (6, (1, 1, 1)), (80, (1, 1, 1)),
                                            (80, (3, 5, 2)), (128, (40, 40, 1))])
def test_plan_dense_cells_bit_exact(channels, cells, device):
    """Tiles with tens of thousands of list entries: the work is cut into
    slices, groups and carries; with exactly representable sums the result
    must equal the oracle bit for bit, whatever the cut."""
    sc = lss_scene.rig(seed=7, height=8, width=22, depth_bins=60, channels=channels)
    sc["desc"] = dict(sc["desc"], minimum=(-60.0, -60.0, -20.0),
                      step=(120.0 / cells[0], 120.0 / cells[1], 40.0 / cells[2]), cells=cells)
    bd, od = _descs(sc["desc"])
    g = _frustum_geometry(sc)
    logits_h, ctx_h = _exact_inputs(sc, channels)
    logits, ctx = _dev(logits_h, device), _dev(ctx_h, device)
    want = ORACLE.lss_lift_pool(logits_h, ctx_h, g, od)
    assert np.count_nonzero(ORACLE.lss_ranks(g, od) >= 0) > 30000
    with bfhip.LssPlan(bd) as plan:
        plan.prepare_geometry(_dev(g, device))
        got = plan.forward(logits, ctx).cpu().numpy()
    assert np.array_equal(got, want)
    geo = _dev(g, device)
    assert np.array_equal(bfhip.lss_lift_pool(logits, ctx, geo, bd).cpu().numpy(), want)


@pytest.mark.parametrize("cells,batches", [((600, 600, 1), 1), ((400, 360, 2), 2)])
def test_plan_keys_of_three_digit_passes(cells, batches, device):
    """Grids whose keys need more than 18 bits take three 9-bit passes of the
    pair sort (360 000 and 576 000 cells, keys up to 2^19 / 2^20): the plan
    must still list every cell's samples in sample order, so the integer
    sums of the exact inputs equal the oracle bit for bit, and the general
    inputs meet the tolerance."""
    sc = lss_scene.rig(seed=9, height=8, width=22, depth_bins=60, channels=8)
    if batches == 2:
        b = lss_scene.rig(seed=10, height=8, width=22, depth_bins=60, channels=8)
        b["extra_rotation"] = lss_scene._rot_z(0.7).reshape(1, 3, 3)
        sc = dict(sc, **{k: np.concatenate([sc[k], b[k]]) for k in
                         ("depth_logits", "context", *lss_scene.CALIBRATION_KEYS)})
    sc["desc"] = dict(sc["desc"], batches=batches, minimum=(-60.0, -60.0, -5.0),
                      step=(120.0 / cells[0], 120.0 / cells[1], 10.0 / cells[2]), cells=cells)
    bd, od = _descs(sc["desc"])
    g = _frustum_geometry(sc)
    assert batches * cells[0] * cells[1] * cells[2] > 1 << 18
    with bfhip.LssPlan(bd) as plan:
        plan.prepare_geometry(_dev(g, device))
        got = plan.forward(_dev(sc["depth_logits"], device), _dev(sc["context"], device))
        _check(got.cpu().numpy(), sc["depth_logits"], sc["context"], g, od,
               f"lss plan {cells} x {batches}")
        logits_h, ctx_h = _exact_inputs(sc, 3)
        exact = plan.forward(_dev(logits_h, device), _dev(ctx_h, device)).cpu().numpy()
    assert np.array_equal(exact, ORACLE.lss_lift_pool(logits_h, ctx_h, g, od))


def test_all_samples_outside_or_non_finite(device):
    sc = SCENES["compact"]
    bd, od = _descs(sc["desc"])
    g = _geometry(sc).copy()
    g[..., 0] = 100.0
    g[0, 0, 0, 0, 0] = np.nan
    g[1, 1, 2, 1, 3] = -np.inf
    logits, ctx = _dev(sc["depth_logits"], device), _dev(sc["context"], device)
    with bfhip.LssPlan(bd) as plan:
        plan.prepare_geometry(_dev(g, device))
        out = plan.forward(logits, ctx).cpu().numpy()
    assert not out.any()
    assert not bfhip.lss_lift_pool(logits, ctx, _dev(g, device), bd).cpu().numpy().any()


def test_unprepared_plan_is_rejected(device):
    bd, _ = _descs(SCENES["compact"]["desc"])
    sc = SCENES["compact"]
    with bfhip.LssPlan(bd) as plan:
        with pytest.raises(bfhip.BfHipError, match="unprepared"):
            plan.forward(_dev(sc["depth_logits"], device), _dev(sc["context"], device))


@pytest.mark.parametrize("name", ["compact", "rig_small", "production"])
def test_stateless_atomic_routes(name, device):
    sc = SCENES[name]
    bd, od = _descs(sc["desc"])
    g = _geometry(sc)
    logits, ctx = _dev(sc["depth_logits"], device), _dev(sc["context"], device)
    geo = _dev(g, device)
    direct = bfhip.lss_lift_pool(logits, ctx, geo, bd).cpu().numpy()
    ranks = bfhip.lss_geometry_to_ranks(geo, bd)
    ranked = bfhip.lss_lift_pool_ranks(logits, ctx, ranks, bd).cpu().numpy()
    for got, route in ((direct, "geometry"), (ranked, "ranks")):
        want = _check(got, sc["depth_logits"], sc["context"], g, od, f"lss atomic {route} {name}")
        if name == "compact":
            assert np.all(np.abs(got - want) <= 2e-6 + 8e-6 * np.abs(want))


def test_plan_forward_graph_replays(device):
    import torch
    sc = SCENES["rig_small"]
    bd, od = _descs(sc["desc"])
    g = _geometry(sc)
    logits, ctx = _dev(sc["depth_logits"], device), _dev(sc["context"], device)
    with bfhip.LssPlan(bd) as plan:
        plan.prepare_geometry(_dev(g, device))
        eager = plan.forward(logits, ctx).clone()
        out = torch.empty_like(eager)
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            plan.forward(logits, ctx, out=out, stream=stream)
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            plan.forward(logits, ctx, out=out)
        for i in range(4):
            out.fill_(float(i) - 7.0)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"graph replay {i} differs"
