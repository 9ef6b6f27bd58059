"""Synthetic lift-splat-shoot inputs (host numpy arrays, float32).

Three scenes, each a dict with the calibration tensors, the frustum, the depth
logits and context, and the ``bf_lss_desc`` fields under ``"desc"``:

``compact(seed)``
    The reference's CPU oracle case (tools/oracle_kernels.py:237-290):
    2 batches x 2 cameras, 4 depth bins, 3 x 5 features, 3 channels, a 6 x 6
    x 4 grid of 2 m cells from (-6, -6, -3), with that file's camera,
    intrinsics, image-augmentation and lidar-augmentation formulas; logits
    and context are seeded normal draws.
``production()``
    The reference's production benchmark inputs (tests/test_cuda_lss.cu:26-63,
    68-104): 1 batch x 6 cameras, 118 depth bins, 32 x 88 features, 80
    channels, a 360 x 360 x 1 grid of 0.3 m cells from (-54, -54, -10);
    logits ((i % 23) - 11) * 0.03, context ((i % 23) - 11) * 0.01, the
    benchmark's spread geometry, and its frustum with identity calibration
    (every sample lands inside the grid).
``rig(seed, height, width)``
    A surround rig in the nuScenes layout: six cameras at yaw 0, +-55, +-110
    and 180 degrees, 1.5 m from the lidar at 1.6 m height, focal length 560 px
    on a 704 x 256 image; depth bins 1.0 + 0.5 k m.  Cells near the vehicle
    collect hundreds of samples, as in real scenes.
"""

from __future__ import annotations

import numpy as np

PRODUCTION = dict(batches=1, cameras=6, depth_bins=118, height=32, width=88, channels=80,
                  minimum=(-54.0, -54.0, -10.0), step=(0.3, 0.3, 20.0), cells=(360, 360, 1))


def _rot_z(angle):
    c, s = np.cos(np.float32(angle)), np.sin(np.float32(angle))
    return np.array([[c, -s, 0.0], [s, c, 0.0], [0.0, 0.0, 1.0]], np.float32)


def compact(seed: int = 0) -> dict:
    b, n, d, h, w, c = 2, 2, 4, 3, 5, 3
    depth = np.broadcast_to(np.arange(1, d + 1, dtype=np.float32).reshape(d, 1, 1), (d, h, w))
    ix = np.broadcast_to(np.linspace(0, 19, w, dtype=np.float32).reshape(1, 1, w), (d, h, w))
    iy = np.broadcast_to(np.linspace(0, 11, h, dtype=np.float32).reshape(1, h, 1), (d, h, w))
    frustum = np.stack((ix, iy, depth), -1).astype(np.float32)
    cam_rot = np.empty((b, n, 3, 3), np.float32)
    cam_trans = np.empty((b, n, 3), np.float32)
    intr = np.empty((b, n, 3, 3), np.float32)
    post_rot = np.empty((b, n, 3, 3), np.float32)
    post_trans = np.empty((b, n, 3), np.float32)
    for bi in range(b):
        for ci in range(n):
            cam_rot[bi, ci] = _rot_z(0.13 * (ci + 1) - 0.04 * bi)
            cam_trans[bi, ci] = (-2.0 + ci * 3.0, -1.0 + bi * 2.0, 0.2 * ci)
            intr[bi, ci] = [[8.0 + ci, 0.0, 9.0], [0.0, 7.0 + bi, 5.0], [0.0, 0.0, 1.0]]
            scale = 0.9 + 0.05 * ci
            post_rot[bi, ci] = [[scale, -0.03, 0.0], [0.02, scale, 0.0], [0.0, 0.0, 1.0]]
            post_trans[bi, ci] = (0.2 * ci, -0.1 * bi, 0.0)
    extra_rot = np.stack([_rot_z(-0.07 + 0.11 * bi) for bi in range(b)])
    extra_trans = np.array([[0.15 * bi, -0.2 * bi, 0.1] for bi in range(b)], np.float32)
    rng = np.random.default_rng(seed)
    return dict(
        desc=dict(batches=b, cameras=n, depth_bins=d, height=h, width=w, channels=c,
                  minimum=(-6.0, -6.0, -3.0), step=(2.0, 2.0, 2.0), cells=(6, 6, 4)),
        frustum=frustum, camera_rotation=cam_rot, camera_translation=cam_trans,
        intrinsics=intr, post_rotation=post_rot, post_translation=post_trans,
        extra_rotation=extra_rot, extra_translation=extra_trans,
        depth_logits=rng.standard_normal((b, n, d, h, w)).astype(np.float32),
        context=rng.standard_normal((b, n, c, h, w)).astype(np.float32))


def _pattern(count, scale):
    i = np.arange(count, dtype=np.int64)
    return (((i % 23) - 11) * np.float32(scale)).astype(np.float32)


def production() -> dict:
    p = PRODUCTION
    n, d, h, w, c = p["cameras"], p["depth_bins"], p["height"], p["width"], p["channels"]
    s = np.arange(n * d * h * w, dtype=np.int64)
    x = s % w
    q = s // w
    y = q % h
    q //= h
    depth = q % d
    cam = (q // d) % 6
    cx = (x * 4 + depth + cam * 13) % 360
    cy = (y * 9 + depth * 3 + cam * 17) % 360
    geometry = np.stack([np.float32(-54.0) + (cx.astype(np.float32) + np.float32(0.5))
                         * np.float32(0.3),
                         np.float32(-54.0) + (cy.astype(np.float32) + np.float32(0.5))
                         * np.float32(0.3),
                         np.zeros(s.size, np.float32)], -1).astype(np.float32)
    f = np.arange(d * h * w, dtype=np.int64)
    fx = f % w
    fq = f // w
    fy = fq % h
    fd = fq // h
    fcx = (fx * 4 + fd) % 360
    fcy = (fy * 9 + fd * 3) % 360
    frustum = np.stack([np.float32(-54.0) + (fcx.astype(np.float32) + np.float32(0.5))
                        * np.float32(0.3),
                        np.float32(-54.0) + (fcy.astype(np.float32) + np.float32(0.5))
                        * np.float32(0.3),
                        np.ones(f.size, np.float32)], -1).astype(np.float32)
    eye = np.broadcast_to(np.eye(3, dtype=np.float32), (1, n, 3, 3)).copy()
    return dict(
        desc=dict(p),
        depth_logits=_pattern(n * d * h * w, 0.03).reshape(1, n, d, h, w),
        context=_pattern(n * c * h * w, 0.01).reshape(1, n, c, h, w),
        geometry=geometry.reshape(1, n, d, h, w, 3),
        frustum=frustum.reshape(d, h, w, 3),
        camera_rotation=eye, intrinsics=eye.copy(), post_rotation=eye.copy(),
        camera_translation=np.zeros((1, n, 3), np.float32),
        post_translation=np.zeros((1, n, 3), np.float32),
        extra_rotation=np.eye(3, dtype=np.float32).reshape(1, 3, 3),
        extra_translation=np.zeros((1, 3), np.float32))


def rig(seed: int = 0, height: int = 32, width: int = 88, depth_bins: int = 118,
        channels: int = 80) -> dict:
    n = 6
    ds = (1.0 + 0.5 * np.arange(depth_bins)).astype(np.float32)
    xs = np.linspace(0, 703, width, dtype=np.float32)
    ys = np.linspace(0, 255, height, dtype=np.float32)
    frustum = np.stack(np.broadcast_arrays(xs.reshape(1, 1, width), ys.reshape(1, height, 1),
                                           ds.reshape(depth_bins, 1, 1)), -1).astype(np.float32)
    # camera axes (x right, y down, z forward) -> lidar axes (x forward, y left, z up)
    base = np.array([[0, 0, 1], [-1, 0, 0], [0, -1, 0]], np.float32)
    yaws = np.deg2rad([0.0, 55.0, -55.0, 180.0, 110.0, -110.0])
    cam_rot = np.stack([_rot_z(a) @ base for a in yaws]).astype(np.float32)[None]
    cam_trans = np.array([[1.5 * np.cos(a), 1.5 * np.sin(a), 1.6] for a in yaws],
                         np.float32)[None]
    intr = np.broadcast_to(np.array([[560.0, 0.0, 352.0], [0.0, 560.0, 140.0],
                                     [0.0, 0.0, 1.0]], np.float32), (1, n, 3, 3)).copy()
    post_rot = np.broadcast_to(np.eye(3, dtype=np.float32), (1, n, 3, 3)).copy()
    post_trans = np.zeros((1, n, 3), np.float32)
    rng = np.random.default_rng(seed)
    return dict(
        desc=dict(PRODUCTION, height=height, width=width, depth_bins=depth_bins,
                  channels=channels),
        frustum=frustum, camera_rotation=cam_rot, camera_translation=cam_trans,
        intrinsics=intr, post_rotation=post_rot, post_translation=post_trans,
        extra_rotation=_rot_z(0.05).reshape(1, 3, 3),
        extra_translation=np.array([[0.2, -0.1, 0.0]], np.float32),
        depth_logits=(2.0 * rng.standard_normal((1, n, depth_bins, height, width))).astype(
            np.float32),
        context=rng.standard_normal((1, n, channels, height, width)).astype(np.float32))


CALIBRATION_KEYS = ("camera_rotation", "camera_translation", "intrinsics", "post_rotation",
                    "post_translation", "extra_rotation", "extra_translation")
