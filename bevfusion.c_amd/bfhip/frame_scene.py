"""Synthetic full frames for the runtime path (host numpy arrays, float32).

``calibration(seed)`` returns the five row-major 4x4 matrix sets of a
``bf_frame_input`` (include/bf_runtime.h) for the surround rig of
``lss_scene.rig`` (six cameras at yaw 0, +-55, +-110, 180 degrees, 1.5 m out
at 1.6 m height, f = 560 px on 704 x 256 images), mutually consistent: the
depth raster projects a lidar point with lidar_to_image = K [R^T | -R^T t]
and the image augmentation, and LSS lifts a pixel back through the inverse
of the same chain.  The image augmentation is a resize by 1 - 0.01 k with a
small crop shift per camera; the lidar augmentation a small yaw and shift.

``frame(seed, points)`` adds images (U[0,1] normalised with the ImageNet mean
and std the reference's YAML fixes) and a LiDAR-like point cloud.
"""

from __future__ import annotations

import numpy as np

from . import bfw

CAMERAS, IMAGE_H, IMAGE_W = 6, 256, 704
_MEAN = np.array([0.485, 0.456, 0.406], np.float32)
_STD = np.array([0.229, 0.224, 0.225], np.float32)


def _rot_z(angle):
    c, s = np.cos(angle), np.sin(angle)
    return np.array([[c, -s, 0.0], [s, c, 0.0], [0.0, 0.0, 1.0]])


def _h(r, t):
    m = np.eye(4)
    m[:3, :3] = r
    m[:3, 3] = t
    return m


def calibration(seed: int = 0) -> dict:
    rng = np.random.default_rng(seed)
    base = np.array([[0, 0, 1], [-1, 0, 0], [0, -1, 0]], np.float64)
    yaws = np.deg2rad([0.0, 55.0, -55.0, 180.0, 110.0, -110.0])
    k = np.array([[560.0, 0.0, 352.0], [0.0, 560.0, 140.0], [0.0, 0.0, 1.0]])
    cam_to_lidar, intrinsics, image_aug, lidar_to_image = [], [], [], []
    for i, a in enumerate(yaws):
        r = _rot_z(a) @ base
        t = np.array([1.5 * np.cos(a), 1.5 * np.sin(a), 1.6])
        cam_to_lidar.append(_h(r, t))
        intrinsics.append(_h(k, np.zeros(3)))
        s = 1.0 - 0.01 * i
        image_aug.append(_h(np.diag([s, s, 1.0]), [rng.uniform(-4, 4), rng.uniform(-3, 3), 0.0]))
        proj = np.eye(4)
        proj[:3, :3] = k @ r.T
        proj[:3, 3] = -(k @ r.T @ t)
        lidar_to_image.append(proj)
    lidar_aug = _h(_rot_z(rng.uniform(-0.05, 0.05)), [rng.uniform(-0.2, 0.2),
                                                       rng.uniform(-0.2, 0.2), 0.0])
    f32 = lambda m: np.ascontiguousarray(np.array(m, np.float32))
    return dict(camera_intrinsics=f32(intrinsics), camera_to_lidar=f32(cam_to_lidar),
                image_augmentation=f32(image_aug), lidar_augmentation=f32(lidar_aug),
                lidar_to_image=f32(lidar_to_image))


def frustum(bins: int = 118, height: int = 32, width: int = 88) -> np.ndarray:
    """The LSS frustum [D,H,W,3] of (pixel x, pixel y, depth): feature columns
    and rows spread evenly over the 704 x 256 image, depth bins 1.0 + 0.5 k m
    (the checkpoint's vtransform.frustum for dbound [1, 60, 0.5])."""
    xs = np.linspace(0.0, IMAGE_W - 1, width, dtype=np.float32)
    ys = np.linspace(0.0, IMAGE_H - 1, height, dtype=np.float32)
    ds = (1.0 + 0.5 * np.arange(bins)).astype(np.float32)
    f = np.stack(np.broadcast_arrays(xs.reshape(1, 1, width), ys.reshape(1, height, 1),
                                     ds.reshape(bins, 1, 1)), -1)
    return np.ascontiguousarray(f, np.float32)


BFI_FIELDS = ("images", "points", "camera_intrinsics", "camera_to_lidar", "image_augmentation",
              "lidar_augmentation", "lidar_to_image")


def write_bfi(frame: dict, path) -> int:
    """Pack a frame as a BFI file (layout in include/bf_frame.h): 128-byte
    little-endian header, then the seven float32 payloads densely in order,
    CRC-32 of the payload in the header.  Returns the file size."""
    import struct
    import zlib
    parts = [np.ascontiguousarray(frame[k], "<f4").tobytes() for k in BFI_FIELDS]
    points = frame["points"].shape[0]
    offsets, at = [], 128
    for part in parts:
        offsets.append(at)
        at += len(part)
    crc = 0
    for part in parts:
        crc = zlib.crc32(part, crc)
    header = struct.pack("<4sIIIQQII7Q", b"BFI1", 1, 128, 0, at, points, crc & 0xffffffff, 0,
                         *offsets)
    header += bytes(128 - len(header))
    with open(path, "wb") as f:
        f.write(header)
        for part in parts:
            f.write(part)
    return at


def images(seed: int) -> np.ndarray:
    raw = bfw.randu(seed, "frame_images", (CAMERAS, IMAGE_H, IMAGE_W, 3))
    return np.ascontiguousarray(((raw - _MEAN) / _STD).transpose(0, 3, 1, 2).astype(np.float32))


def frame(seed: int = 0, points: int = 60000, sweeps: int = 1) -> dict:
    out = calibration(seed)
    out["images"] = images(seed)
    out["points"] = bfw.synthetic_points(seed, points, sweeps=sweeps)
    return out
