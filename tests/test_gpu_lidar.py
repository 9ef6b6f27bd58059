"""LiDAR side on the GPU against the CPU oracle (oracle/src/lidar.c, itself
pinned bit-exact to the reference's depth_raster.c, voxel.c and
lidar_backbone.c and to float64 torch convolutions).

Follows the reference's tests/test_cuda_depth_raster.cu, test_cuda_voxel.cu
and test_cuda_lidar.cu: each context against the CPU path on the same
synthetic frame.  Bars:
  * depth raster: bit-exact (the projection keeps the CPU's unfused operation
    order; "later point wins" is an order-free integer max);
  * voxeliser: coordinates, voxel count and MeanVFE means bit-exact, in the
    CPU's first-encounter voxel order, through both caps;
  * sparse encoder: the dense BEV within the north-star tolerance (rel-L2
    <= 1e-2, max-abs <= 5e-2 RMS) -- its GEMMs take split fp16 operands
    (hi + lo) with fp32 accumulation -- and zero at every cell where the
    oracle's BEV has no site;
  * the three contexts captured in one HIP graph replay bit-identically to
    their eager launches (no memset or allocation inside).
"""

import numpy as np
import pytest

import bfhip
import oracle
from bfhip import bfw, frame_scene
from util import assert_close, clustered_sites

pytestmark = pytest.mark.gpu


def _t(a, device, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).to(device)
    return t if dtype is None else t.to(dtype)


def _raster_oracle(points, cal):
    pts = np.concatenate([np.zeros((len(points), 1), np.float32), points], 1)
    return oracle.Oracle("port").depth_raster(pts, cal["lidar_augmentation"],
                                              cal["lidar_to_image"], cal["image_augmentation"],
                                              6, 256, 704)[0]


def _raster_gpu(r, points, cal, device):
    print(f"[case] depth raster P={len(points)}", flush=True)
    out = r.forward(_t(points, device), _t(cal["lidar_augmentation"], device),
                    _t(cal["lidar_to_image"], device), _t(cal["image_augmentation"], device))
    return out.cpu().numpy()


def test_depth_raster_bit_exact(device):
    cal = frame_scene.calibration(3)
    with bfhip.DepthRaster(250000) as r:
        assert r.resident_bytes() > 0
        for seed, n in ((3, 20000), (4, 250000), (5, 777)):
            pts = bfw.synthetic_points(seed, n)
            got, want = _raster_gpu(r, pts, cal, device), _raster_oracle(pts, cal)
            assert np.array_equal(got, want), f"P={n}: depth differs at {np.argwhere(got != want)[:5]}"
            assert (want > 0).sum() > min(n, 2000) // 4
        # Empty cloud: the owner words were cleared by the previous call.
        empty = np.zeros((0, 5), np.float32)
        assert not _raster_gpu(r, empty, cal, device).any()


def test_depth_raster_known_answers(device):
    cal = frame_scene.calibration(0)
    eye = np.eye(4, dtype=np.float32)
    cam0 = cal["camera_to_lidar"][0]
    far = cam0[:3, :3] @ np.array([0.0, 0.0, 10.0], np.float32) + cam0[:3, 3]
    near = cam0[:3, :3] @ np.array([0.0, 0.0, 5.0], np.float32) + cam0[:3, 3]
    c = dict(cal, lidar_augmentation=eye,
             image_augmentation=np.broadcast_to(eye, (6, 4, 4)).copy())
    pts = np.array([[*far, 0, 0], [*near, 0, 0]], np.float32)
    with bfhip.DepthRaster(16) as r:
        d = _raster_gpu(r, pts, c, device)
        assert d[0, 140, 352] == pytest.approx(5.0, rel=1e-5) and (d > 0).sum() == 1
        d = _raster_gpu(r, pts[::-1].copy(), c, device)
        assert d[0, 140, 352] == pytest.approx(10.0, rel=1e-5) and (d > 0).sum() == 1
        # A singular lidar augmentation leaves the image zero.
        assert not _raster_gpu(r, pts, dict(c, lidar_augmentation=np.zeros((4, 4), np.float32)),
                               device).any()


def _voxel_gpu(vox, points, device):
    import torch
    print(f"[case] voxelize P={len(points)} V={vox.config.max_voxels}", flush=True)
    coords, means, count = vox.forward(_t(points, device))
    torch.cuda.synchronize()
    n = int(count.item())
    return coords[:n].cpu().numpy(), means[:n].cpu().numpy(), n


@pytest.mark.parametrize("points,max_voxels", [(30000, 500), (30000, 40000), (250000, 160000),
                                               (1, 10)])
def test_voxelize_bit_exact(device, points, max_voxels):
    pts = bfw.synthetic_points(5, points) if points > 1 else np.array(
        [[1.0, 2.0, 0.5, 0.3, 0.0]], np.float32)
    cfg = bfhip.voxel_config(max_voxels)
    o = oracle.Oracle("port")
    vx, oc, on, st = o.voxelize(pts, oracle.voxel_config(max_voxels))
    om = o.mean_vfe(vx, on)
    with bfhip.Voxelizer(cfg, 250000) as vox:
        assert vox.resident_bytes() > 0
        gc, gm, n = _voxel_gpu(vox, pts, device)
        assert n == len(oc)
        assert np.array_equal(gc, oc)
        assert np.array_equal(gm, om)
        if max_voxels == 500:
            assert st.dropped_voxel_capacity > 0
        # repeat, then an empty cloud
        gc2, gm2, n2 = _voxel_gpu(vox, pts, device)
        assert n2 == n and np.array_equal(gc2, gc) and np.array_equal(gm2, gm)
        assert _voxel_gpu(vox, np.zeros((0, 5), np.float32), device)[2] == 0


def test_voxelize_known_answers(device):
    cfg = bfhip.voxel_config(2, max_points=2)
    p = np.array([[0.01, 0.01, 0.01, 1, 0], [10.0, 0.0, 0.0, 2, 0], [0.02, 0.02, 0.02, 3, 0],
                  [20.0, 0.0, 0.0, 4, 0], [0.03, 0.03, 0.03, 5, 0]], np.float32)
    with bfhip.Voxelizer(cfg, 8) as vox:
        coords, means, n = _voxel_gpu(vox, p, device)
    assert n == 2 and coords.tolist() == [[0, 25, 720, 720], [0, 25, 720, 853]]
    assert means[0, 3] == 2.0 and means[1, 3] == 2.0


@pytest.fixture(scope="module")
def lidar_path(tmp_path_factory):
    return bfw.write_lidar_backbone(tmp_path_factory.mktemp("lidar") / "lidar.bfw", seed=4,
                                    mode="fan_in", gain=1.2)


def _backbone_oracle(path, coords, feats, d, h, w):
    o = oracle.Oracle("port")
    with o.open_model(path) as m:
        return o.lidar_backbone(m, coords, feats, d, h, w, capacity=max(8 * len(coords), 4096))


def _check_bev(got, want, tag):
    assert got.shape == want.shape, tag
    # Cells with a site (some channel non-zero): the GPU adds none.
    gm, wm = (got != 0).any(axis=1), (want != 0).any(axis=1)
    assert wm.sum() > 0 and not (gm & ~wm).any(), f"{tag}: output at cells without a site"
    assert_close(got, want, tag)


def test_lidar_backbone_small_grid(device, lidar_path):
    import torch
    coords = clustered_sites(7, 900, 41, 96, 96)
    feats = np.random.default_rng(8).standard_normal((len(coords), 5)).astype(np.float32)
    want = _backbone_oracle(lidar_path, coords, feats, 41, 96, 96)
    with bfhip.Model(lidar_path) as m:
        net = bfhip.LidarBackbone(m, 1, 41, 96, 96, 20000)
    assert net.resident_bytes() > 0
    c, f = _t(coords, device), _t(feats, device)
    print(f"[case] lidar backbone 41x96x96 N={len(coords)}", flush=True)
    got = net.forward(c, f, len(coords)).cpu().numpy()
    _check_bev(got, want, "41x96x96")
    # Device count, a repeat and a different, smaller input: the index grids
    # are clean between forwards.
    cnt = torch.tensor([len(coords)], dtype=torch.int32, device=device)
    again = net.forward(c, f, cnt).cpu().numpy()
    assert np.array_equal(again, got)
    half = coords[: len(coords) // 2]
    want2 = _backbone_oracle(lidar_path, half, feats[: len(half)], 41, 96, 96)
    got2 = net.forward(_t(half, device), _t(feats[: len(half)], device), len(half)).cpu().numpy()
    _check_bev(got2, want2, "41x96x96 half")
    net.close()


def test_lidar_pipeline_production_grid(device, lidar_path):
    """Points -> GPU voxeliser -> GPU encoder (device voxel count) at the
    production 41 x 1440 x 1440 grid against the oracle chain."""
    import torch
    pts = bfw.synthetic_points(11, 100000, sweeps=10)
    cfg = bfhip.voxel_config(160000)
    o = oracle.Oracle("port")
    vx, oc, on, _ = o.voxelize(pts, oracle.voxel_config(160000))
    want = _backbone_oracle(lidar_path, oc, o.mean_vfe(vx, on), 41, 1440, 1440)
    assert want.shape == (1, 128, 2, 180, 180)
    with bfhip.Voxelizer(cfg, 300000) as vox, bfhip.Model(lidar_path) as m:
        net = bfhip.LidarBackbone(m, 1, 41, 1440, 1440, 160000)
        print(f"[case] lidar pipeline 41x1440x1440 P={len(pts)}", flush=True)
        coords, means, count = vox.forward(_t(pts, device))
        got = net.forward(coords, means, count)
        torch.cuda.synchronize()
        assert int(count.item()) == len(oc)
        _check_bev(got.cpu().numpy(), want, "production")
        net.close()


def test_lidar_pipeline_reference_stress_frame(device, lidar_path):
    """The reference's own stress frame (tests/test_cuda_lidar.cu: 100k
    points, two per voxel, 50k voxels; level 1 holds 155 985 sites, just
    under the runtime's 160 000 capacity) through the GPU voxeliser and
    encoder against the oracle chain."""
    import torch
    pts = bfw.stress_points(100000)
    o = oracle.Oracle("port")
    vx, oc, on, _ = o.voxelize(pts, oracle.voxel_config(160000))
    assert len(oc) == 50000 and np.all(on == 2)
    om = o.mean_vfe(vx, on)
    want = _backbone_oracle(lidar_path, oc, om, 41, 1440, 1440)
    with bfhip.Voxelizer(bfhip.voxel_config(160000), 100000) as vox, bfhip.Model(lidar_path) as m:
        net = bfhip.LidarBackbone(m, 1, 41, 1440, 1440, 160000)
        print("[case] lidar stress frame 100k points", flush=True)
        coords, means, count = vox.forward(_t(pts, device))
        got = net.forward(coords, means, count)
        torch.cuda.synchronize()
        n = int(count.item())
        assert n == 50000
        assert np.array_equal(coords[:n].cpu().numpy(), oc)
        assert np.array_equal(means[:n].cpu().numpy(), om)
        _check_bev(got.cpu().numpy(), want, "stress")
        net.close()


def test_lidar_backbone_capacity_overflow(device, lidar_path):
    """Scattered sites whose strided images outnumber `sparse_capacity` at
    level 1: the forward drops the sites beyond the capacity in cell order
    (the reference GPU path drops an arbitrary subset), stays finite and
    repeats bit for bit; with room for every site it matches the oracle."""
    import torch
    rng = np.random.default_rng(12)
    cells = rng.choice(41 * 96 * 96, size=400, replace=False)
    coords = np.stack([np.zeros(400, np.int64), cells // (96 * 96), cells // 96 % 96, cells % 96],
                      1).astype(np.int32)
    feats = rng.standard_normal((400, 5)).astype(np.float32)
    c, f = _t(coords, device), _t(feats, device)
    with bfhip.Model(lidar_path) as m:
        small = bfhip.LidarBackbone(m, 1, 41, 96, 96, 1000)
        roomy = bfhip.LidarBackbone(m, 1, 41, 96, 96, 20000)
    print("[case] lidar capacity overflow 400 sites, capacity 1000", flush=True)
    a = small.forward(c, f, 400).cpu().numpy()
    b = small.forward(c, f, 400).cpu().numpy()
    full = roomy.forward(c, f, 400).cpu().numpy()
    assert np.isfinite(a).all() and np.array_equal(a, b)
    assert (a != 0).any() and not np.array_equal(a, full)
    _check_bev(full, _backbone_oracle(lidar_path, coords, feats, 41, 96, 96), "scattered")
    small.close()
    roomy.close()


def test_lidar_graph_replay(device, lidar_path):
    """Raster + voxeliser + encoder captured in one graph; every replay, with
    eager work and synchronisation in between, equals the eager frame."""
    import torch
    cal = frame_scene.calibration(2)
    frames = [bfw.synthetic_points(s, 30000, sweeps=3) for s in (21, 22)]
    raster = bfhip.DepthRaster(40000)
    vox = bfhip.Voxelizer(bfhip.voxel_config(160000), 40000)
    with bfhip.Model(lidar_path) as m:
        net = bfhip.LidarBackbone(m, 1, 41, 1440, 1440, 160000)
    pts = _t(frames[0], device)
    mats = [_t(cal[k], device) for k in ("lidar_augmentation", "lidar_to_image",
                                         "image_augmentation")]
    depth = torch.empty((6, 256, 704), device=device)
    coords = torch.empty((160000, 4), dtype=torch.int32, device=device)
    means = torch.empty((160000, 5), device=device)
    count = torch.empty((1,), dtype=torch.int32, device=device)
    bev = torch.empty(net.out_shape, device=device)
    stream = torch.cuda.Stream()

    def frame():
        raster.forward(pts, *mats, out=depth, stream=stream)
        vox.forward(pts, coords, means, count, stream=stream)
        net.forward(coords, means, count, out=bev, stream=stream)

    def snap():
        stream.synchronize()
        return depth.cpu().numpy().copy(), count.item(), bev.cpu().numpy().copy()

    print("[case] lidar graph replay", flush=True)
    eager = []
    with torch.cuda.stream(stream):
        for f in frames:
            pts.copy_(_t(f, device))
            frame()
            eager.append(snap())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            frame()
        for rep in range(4):
            k = rep % 2
            pts.copy_(_t(frames[k], device))
            graph.replay()
            got = snap()
            assert np.array_equal(got[0], eager[k][0]), f"replay {rep}: depth differs"
            assert got[1] == eager[k][1], f"replay {rep}: voxel count differs"
            assert np.array_equal(got[2], eager[k][2]), f"replay {rep}: BEV differs"
            frame()  # eager work between replays
            assert np.array_equal(snap()[2], eager[k][2])
    for ctx in (raster, vox, net):
        ctx.close()
