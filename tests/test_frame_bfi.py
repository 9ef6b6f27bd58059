"""BFI frame files (include/bf_frame.h, bevfusion.c_amd/csrc/bfi_frame.c).

Follows the reference's tests/test_frame.c: a packed frame opens and its
view holds the packed values; a payload byte changed after packing (CRC), a
header field, a payload offset, a truncated file and a non-finite value are
each rejected.  The packer (bfhip.frame_scene.write_bfi) and the reader are
pinned against the reference's own reader (src/frame.c compiled into
oracle/_ref): it opens the same files and sees the same values, and rejects
the same corruptions.
"""

import ctypes as C
import struct
import zlib

import numpy as np
import pytest

import bfhip
import oracle
from bfhip import frame_scene


@pytest.fixture(scope="module")
def frame():
    f = frame_scene.frame(seed=2, points=777)
    f["points"] = np.nan_to_num(f["points"], nan=0.25)  # BFI holds finite values only
    return f


def _ref_open(path):
    """The reference's bf_frame_open (oracle/_ref) -> view or None."""
    lib = C.CDLL(str(oracle.LIBS["ref"]))
    lib.bf_frame_open.argtypes = [C.c_char_p, C.POINTER(C.c_void_p), C.c_char_p, C.c_size_t]
    lib.bf_frame_input_view.restype = C.POINTER(oracle.FrameInput)
    lib.bf_frame_input_view.argtypes = [C.c_void_p]
    lib.bf_frame_close.argtypes = [C.c_void_p]
    h, err = C.c_void_p(), C.create_string_buffer(256)
    if not lib.bf_frame_open(str(path).encode(), C.byref(h), err, 256):
        return None
    v = lib.bf_frame_input_view(h).contents
    out = _arrays(v)
    lib.bf_frame_close(h)
    return out


def _arrays(v):
    shapes = dict(camera_images=(6, 3, 256, 704), points=(v.point_count, 5),
                  camera_intrinsics_6x16=(6, 4, 4), camera_to_lidar_6x16=(6, 4, 4),
                  image_augmentation_6x16=(6, 4, 4), lidar_augmentation_16=(4, 4),
                  lidar_to_image_6x16=(6, 4, 4))
    out = {}
    for name, shape in shapes.items():
        n = int(np.prod(shape))
        ptr = C.cast(getattr(v, name), C.POINTER(C.c_float * n)).contents
        out[name] = np.frombuffer(ptr, np.float32, n).reshape(shape).copy()
    return out


EXPECT = dict(camera_images="images", points="points", camera_intrinsics_6x16="camera_intrinsics",
              camera_to_lidar_6x16="camera_to_lidar",
              image_augmentation_6x16="image_augmentation",
              lidar_augmentation_16="lidar_augmentation", lidar_to_image_6x16="lidar_to_image")


def _same(got, frame):
    for name, key in EXPECT.items():
        assert np.array_equal(got[name], np.asarray(frame[key], np.float32).reshape(got[name].shape)), name


def test_round_trip(tmp_path, frame):
    path = tmp_path / "f.bfi"
    size = frame_scene.write_bfi(frame, path)
    assert path.stat().st_size == size == 128 + 4 * (6 * 3 * 256 * 704 + 777 * 5 + 4 * 96 + 16)
    with bfhip.FrameFile(path) as f:
        assert f.bytes() == size and f.input.point_count == 777
        _same(_arrays(f.input), frame)
    if oracle.available("ref"):
        _same(_ref_open(path), frame)


def _rewrite(raw, path, fix_crc=True):
    raw = bytearray(raw)
    if fix_crc:
        struct.pack_into("<I", raw, 32, zlib.crc32(bytes(raw[128:])) & 0xffffffff)
    path.write_bytes(bytes(raw))
    return path


@pytest.mark.parametrize("case", ["payload_byte", "magic", "version", "size_field",
                                  "offset", "zero_points", "truncated", "nan"])
def test_rejects_corruption(tmp_path, frame, case):
    path = tmp_path / "f.bfi"
    frame_scene.write_bfi(frame, path)
    raw = bytearray(path.read_bytes())
    bad = tmp_path / "bad.bfi"
    if case == "payload_byte":   # CRC no longer matches
        raw[200] ^= 1
        _rewrite(raw, bad, fix_crc=False)
    elif case == "magic":
        raw[0:4] = b"BFI2"
        _rewrite(raw, bad)
    elif case == "version":
        struct.pack_into("<I", raw, 4, 2)
        _rewrite(raw, bad)
    elif case == "size_field":
        struct.pack_into("<Q", raw, 16, len(raw) + 4)
        _rewrite(raw, bad)
    elif case == "offset":       # non-canonical points offset
        struct.pack_into("<Q", raw, 48, struct.unpack_from("<Q", raw, 48)[0] + 4)
        _rewrite(raw, bad)
    elif case == "zero_points":
        struct.pack_into("<Q", raw, 24, 0)
        _rewrite(raw, bad)
    elif case == "truncated":
        _rewrite(raw[:-4], bad)
    elif case == "nan":          # CRC-valid, non-finite point
        off = struct.unpack_from("<Q", raw, 48)[0]
        struct.pack_into("<f", raw, off, float("nan"))
        _rewrite(raw, bad)
    with pytest.raises(bfhip.BfHipError):
        bfhip.FrameFile(bad)
    if oracle.available("ref"):
        assert _ref_open(bad) is None
