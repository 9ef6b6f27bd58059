"""CPU checks of the LiDAR-side oracle (oracle/src/lidar.c).

Pinned by (a) the reference's own src/depth_raster.c, src/voxel.c,
src/kernels_ref.c and src/lidar_backbone.c compiled as-is (oracle/_ref):
bit-identical depth images, voxels / coordinates / counts / statistics,
MeanVFE features, sparse-conv outputs and backbone BEV on the scalar path;
(b) float64 torch for the sparse convolution (a submanifold conv is the dense
F.conv3d read at the input sites; a strided one is the dense conv at every
site some input reaches, the rest of its output being exactly zero), so a
wrong tap order, stride, padding or weight layout fails; (c) known answers of
the raster (a point on a camera's axis lands on its principal point; a later
point wins a shared pixel) and the voxeliser (first-encounter order, the
per-voxel point cap and the voxel cap).
"""

import ctypes as C

import numpy as np
import pytest

import oracle
from bfhip import bfw, frame_scene
from util import clustered_sites as _sites

pytestmark = []


def _ref_or_skip():
    if not oracle.available("ref_scalar"):
        pytest.skip("reference CPU sources are not present to build oracle/_ref")


def _both(fn):
    """fn(oracle) on the scalar port and the scalar reference build."""
    out = []
    with oracle.scalar_env():
        for flavour in ("port_scalar", "ref_scalar"):
            out.append(fn(oracle.Oracle(flavour)))
    return out


def _batched(points):
    return np.concatenate([np.zeros((points.shape[0], 1), np.float32), points], 1)


def test_depth_raster_bit_exact_with_reference():
    _ref_or_skip()
    cal = frame_scene.calibration(3)
    pts = _batched(bfw.synthetic_points(3, 20000))
    a, b = _both(lambda o: o.depth_raster(pts, cal["lidar_augmentation"], cal["lidar_to_image"],
                                          cal["image_augmentation"], 6, 256, 704))
    assert np.array_equal(a, b)
    assert (a > 0).sum() > 2000  # the cloud is visible in the images


def test_depth_raster_known_answers():
    o = oracle.Oracle("port")
    cal = frame_scene.calibration(0)
    eye = np.eye(4, dtype=np.float32)
    l2i = cal["lidar_to_image"]
    cam0 = cal["camera_to_lidar"][0]
    # A point 10 m down camera 0's optical axis, identity augmentations.
    axis = cam0[:3, :3] @ np.array([0.0, 0.0, 10.0], np.float32) + cam0[:3, 3]
    pts = np.array([[0.0, *axis, 0.5, 0.0]], np.float32)
    aug = np.broadcast_to(eye, (6, 4, 4)).copy()
    d = o.depth_raster(pts, eye, l2i, aug, 6, 256, 704)
    assert d[0, 0, 140, 352] == pytest.approx(10.0, rel=1e-5)
    assert (d > 0).sum() == 1
    # Two points hitting one pixel: the later one wins.
    near = cam0[:3, :3] @ np.array([0.0, 0.0, 5.0], np.float32) + cam0[:3, 3]
    pts2 = np.array([[0.0, *axis, 0, 0], [0.0, *near, 0, 0]], np.float32)
    d2 = o.depth_raster(pts2, eye, l2i, aug, 6, 256, 704)
    assert d2[0, 0, 140, 352] == pytest.approx(5.0, rel=1e-5)
    d3 = o.depth_raster(pts2[::-1].copy(), eye, l2i, aug, 6, 256, 704)
    assert d3[0, 0, 140, 352] == pytest.approx(10.0, rel=1e-5)


@pytest.mark.parametrize("max_voxels", [500, 40000])
def test_voxelize_bit_exact_with_reference(max_voxels):
    _ref_or_skip()
    pts = bfw.synthetic_points(5, 30000)
    cfg = oracle.voxel_config(max_voxels)
    (va, ca, na, sa), (vb, cb, nb, sb) = _both(lambda o: o.voxelize(pts, cfg))
    assert ca.shape == cb.shape and np.array_equal(ca, cb) and np.array_equal(na, nb)
    for v, n in ((va, na), (vb, nb)):
        for i in range(v.shape[0]):
            v[i, n[i]:] = 0  # rows beyond the count are zeroed by both
    assert np.array_equal(va, vb)
    assert [getattr(sa, f) for f, _ in sa._fields_] == [getattr(sb, f) for f, _ in sb._fields_]
    if max_voxels == 500:
        assert sa.dropped_voxel_capacity > 0 and ca.shape[0] == 500
    assert sa.dropped_point_capacity > 0 and sa.rejected_out_of_range >= 2
    assert sa.rejected_nonfinite >= 1
    fa, fb = _both(lambda o: o.mean_vfe(va, na))
    assert np.array_equal(fa, fb)


def test_voxelize_known_answers():
    o = oracle.Oracle("port")
    cfg = oracle.voxel_config(2, max_points=2)
    p = np.array([[0.01, 0.01, 0.01, 1, 0],     # voxel A
                  [10.0, 0.0, 0.0, 2, 0],       # voxel B
                  [0.02, 0.02, 0.02, 3, 0],     # A again
                  [20.0, 0.0, 0.0, 4, 0],       # voxel C: over the voxel cap
                  [0.03, 0.03, 0.03, 5, 0]],    # A, over the point cap
                 np.float32)
    vox, coords, counts, st = o.voxelize(p, cfg)
    assert coords.tolist() == [[0, 25, 720, 720], [0, 25, 720, 853]]
    assert counts.tolist() == [2, 1]
    assert vox[0, :, 3].tolist() == [1, 3] and vox[1, 0, 3] == 2
    assert st.dropped_voxel_capacity == 1 and st.dropped_point_capacity == 1
    assert o.mean_vfe(vox, counts)[0, 3] == 2.0


def _dense_conv(coords, feats, weight, bias, d, h, w, stride, pad):
    """float64 F.conv3d of the scattered features; weight [kd,kh,kw,ci,co]."""
    import torch
    import torch.nn.functional as F
    ci = feats.shape[1]
    x = torch.zeros((1, ci, d, h, w), dtype=torch.float64)
    c = torch.from_numpy(coords.astype(np.int64))
    x[0, :, c[:, 1], c[:, 2], c[:, 3]] = torch.from_numpy(feats.astype(np.float64)).T
    wt = torch.from_numpy(weight.astype(np.float64)).permute(4, 3, 0, 1, 2).contiguous()
    b = None if bias is None else torch.from_numpy(bias.astype(np.float64))
    return F.conv3d(x, wt, b, stride=stride, padding=pad)[0].numpy()


@pytest.mark.parametrize("case", [
    dict(k=(3, 3, 3), s=(1, 1, 1), p=(1, 1, 1), subm=1, ci=5, co=7),
    dict(k=(3, 3, 3), s=(2, 2, 2), p=(1, 1, 1), subm=0, ci=6, co=4),
    dict(k=(3, 3, 3), s=(2, 2, 2), p=(0, 1, 1), subm=0, ci=3, co=5),
    dict(k=(3, 1, 1), s=(2, 1, 1), p=(0, 0, 0), subm=0, ci=4, co=6)])
def test_sparse_conv3d_against_reference_and_torch(case):
    d, h, w = 9, 14, 12
    coords = _sites(1, 120, d, h, w)
    rng = np.random.default_rng(2)
    feats = rng.standard_normal((len(coords), case["ci"])).astype(np.float32)
    weight = rng.standard_normal((*case["k"], case["ci"], case["co"])).astype(np.float32)
    bias = rng.standard_normal(case["co"]).astype(np.float32)
    desc = oracle.SparseDesc(1, d, h, w, case["ci"], case["co"], *case["k"], *case["s"],
                             *case["p"], 1, 1, 1, case["subm"])
    o = oracle.Oracle("port")
    oc, of = o.sparse_conv3d(coords, feats, weight, bias, desc, 4000)
    keys = ((oc[:, 1].astype(np.int64) * 1000 + oc[:, 2]) * 1000 + oc[:, 3])
    assert np.all(np.diff(keys) > 0)  # unique, ascending (batch, z, y, x)
    ref = _dense_conv(coords, feats, weight, bias, d, h, w, case["s"], case["p"])
    got = ref[:, oc[:, 1], oc[:, 2], oc[:, 3]].T
    np.testing.assert_allclose(of, got, rtol=1e-5, atol=1e-5)
    if case["subm"]:
        assert sorted(map(tuple, oc.tolist())) == sorted(map(tuple, coords.tolist()))
    else:
        reach = _dense_conv(coords, np.ones((len(coords), 1), np.float32),
                            np.ones((*case["k"], 1, 1), np.float32), None, d, h, w, case["s"],
                            case["p"])[0]
        assert len(oc) == int((reach > 0).sum())
    if oracle.available("ref_scalar"):
        (ra, fa), (rb, fb) = _both(lambda q: q.sparse_conv3d(coords, feats, weight, bias, desc,
                                                              4000))
        assert np.array_equal(ra, rb) and np.array_equal(fa, fb)


def test_lidar_backbone_bit_exact_with_reference(tmp_path):
    _ref_or_skip()
    path = bfw.write_lidar_backbone(tmp_path / "lidar.bfw", seed=4, mode="fan_in", gain=1.2)
    coords = _sites(7, 900, 41, 96, 96)
    feats = np.random.default_rng(8).standard_normal((len(coords), 5)).astype(np.float32)

    def run(o):
        with o.open_model(path) as m:
            return o.lidar_backbone(m, coords, feats, 41, 96, 96, capacity=20000)

    a, b = _both(run)
    assert a.shape == (1, 128, 2, 12, 12)
    assert np.array_equal(a, b)
    assert np.count_nonzero(a) > 0
