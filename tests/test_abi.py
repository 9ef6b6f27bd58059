"""C-ABI boundary checks that need no GPU.

libbfhip.so must load, export every entry point declared in include/*.h, and
reject invalid contracts before launching anything (reference
src/cuda_ops.cu:150-170,192-196; cuda_swin.cu:272-273; cuda_camera.cu:288-290;
cuda_lss.cu:50-61,617-634,790-797; cuda_bev_stage.cu:222-225,320-322;
cuda_transfusion.cu:274-276,329-333,402-407; tests/test_cuda_ops.cu:164-174).
"""

import ctypes as C
import pathlib
import re
import shutil
import subprocess

import pytest

import bfhip

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADERS = ["bf_cuda_ops.h", "bf_cuda_swin.h", "bf_cuda_camera.h", "bf_cuda.h", "bf_cuda_bev.h",
           "bf_cuda_transfusion.h", "bf_cuda_depth_raster.h", "bf_cuda_voxel.h",
           "bf_cuda_lidar.h", "bf_cuda_runtime.h", "bfhip_profile.h", "bfhip_debug.h"]
MODEL_HEADERS = ["bf_model.h", "bf_frame.h"]  # host readers in libbfmodel.so


def declared(header):
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b((?:bf|bfhip)_[a-z0-9_]+)\s*\(", text))


def test_every_declared_entry_point_is_exported():
    lib = bfhip.hip_lib()
    names = set().union(*(declared(h) for h in HEADERS))
    assert len(names) == 64
    assert names == set(bfhip.SIGNATURES)
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    model = bfhip.model_lib()
    host = set().union(*(declared(h) for h in MODEL_HEADERS))
    assert host == set(bfhip.MODEL_SIGNATURES)
    assert all(hasattr(model, n) for n in host)


def _err():
    return C.create_string_buffer(256)


def test_conv_rejects_invalid_and_oversized():
    lib = bfhip.hip_lib()
    e = _err()
    zero = bfhip.ConvDesc()
    assert lib.bf_cuda_conv2d_f32(C.byref(zero), None, None, None, None, None, e, 256) == 0
    assert b"invalid" in e.value
    big = 2147483647
    over = bfhip.ConvDesc(big, 1, 1, big, big, 1, 1, 1, 1, 0, 0, big, big, 0, 0)
    s = C.c_void_p(1)
    assert lib.bf_cuda_conv2d_f32(C.byref(over), s, s, None, s, None, e, 256) == 0
    assert b"too large" in e.value
    bad_relu = bfhip.ConvDesc(1, 1, 1, 4, 4, 1, 1, 1, 1, 0, 0, 4, 4, 0, 2)
    assert lib.bf_cuda_conv2d_f32(C.byref(bad_relu), s, s, None, s, None, e, 256) == 0
    # NULL / zero-capacity error buffers are allowed.
    assert lib.bf_cuda_conv2d_f32(C.byref(zero), None, None, None, None, None, None, 0) == 0


def test_gemm_rejects_invalid():
    lib = bfhip.hip_lib()
    e = _err()
    s = C.c_void_p(1)
    assert lib.bf_cuda_gemm_f32(s, s, None, s, 0, 4, 4, 0, None, e, 256) == 0
    assert lib.bf_cuda_gemm_f32(s, s, None, s, 4, 4, 4, 2, None, e, 256) == 0
    assert lib.bf_cuda_gemm_f32(None, s, None, s, 4, 4, 4, 0, None, e, 256) == 0
    assert b"invalid" in e.value


def test_contexts_reject_invalid_contracts(tmp_path):
    from bfhip import bfw
    lib = bfhip.hip_lib()
    e = _err()
    out = C.c_void_p()
    assert not lib.bf_cuda_swin_create(None, 6, 256, 704, C.byref(out), e, 256)
    path = tmp_path / "x.bfw"
    bfw.write_bfw([("x", bfw.randn(0, "x", (4,)))], path)
    with bfhip.Model(path) as m:
        assert not lib.bf_cuda_swin_create(m.handle, 6, 258, 704, C.byref(out), e, 256)
        assert b"invalid" in e.value
        assert not lib.bf_cuda_swin_create(m.handle, 0, 256, 704, C.byref(out), e, 256)
        assert not lib.bf_cuda_camera_neck_create(m.handle, 6, 32, 88, 361, 360, C.byref(out),
                                                  e, 256)
        assert b"invalid" in e.value
    assert out.value is None
    assert lib.bf_cuda_swin_resident_bytes(None) == 0
    assert lib.bf_cuda_camera_neck_resident_bytes(None) == 0
    lib.bf_cuda_swin_destroy(None)
    lib.bf_cuda_camera_neck_destroy(None)
    s = C.c_void_p(1)
    assert not lib.bf_cuda_swin_forward(None, s, s, s, s, None, e, 256)
    assert not lib.bf_cuda_camera_downsample_forward(None, s, s, None, e, 256)
    assert not lib.bf_cuda_camera_neck_forward(None, s, s, s, s, s, s, None, e, 256)


def test_index_probes_reject_invalid():
    lib = bfhip.hip_lib()
    e = _err()
    s = C.c_void_p(1)
    assert lib.bfhip_debug_window_map(1, 7, 7, 7, s, s, None, e, 256) == 0
    assert b"invalid" in e.value
    assert lib.bfhip_debug_window_map(0, 7, 7, 3, s, s, None, e, 256) == 0
    assert lib.bfhip_debug_window_map(1, 7, 7, 3, None, s, None, e, 256) == 0
    # channels must be 32 per head
    assert lib.bfhip_debug_window_attention(s, s, s, s, 1, 7, 7, 64, 3, 0, None, e, 256) == 0
    assert b"invalid" in e.value
    assert lib.bfhip_debug_window_attention(s, s, s, s, 1, 7, 7, 96, 3, 7, None, e, 256) == 0
    assert lib.bfhip_debug_window_attention(s, s, s, s, 70000, 7000, 7000, 96, 3, 3, None, e,
                                            256) == 0
    assert b"too large" in e.value
    assert lib.bfhip_debug_window_attention(s, s, s, s, 1, 7, 7, 96, 3, 3, None, e, 256) == 0
    assert b"16-byte aligned" in e.value
    # The no-allocation variant shares the contract and bounds the head count
    # by its static array; both are checked before any HIP call.
    noalloc = lib.bfhip_debug_window_attention_noalloc
    assert noalloc(s, s, s, s, 1, 7, 7, 64, 3, 0, None, e, 256) == 0
    assert b"invalid" in e.value
    assert noalloc(s, s, s, s, 70000, 7000, 7000, 96, 3, 3, None, e, 256) == 0
    assert b"too large" in e.value
    aligned = C.c_void_p(256)
    assert noalloc(aligned, aligned, aligned, aligned, 1, 7, 7, 32 * 33, 33, 3, None, e, 256) == 0
    assert b"at most 32 heads" in e.value


def test_lss_entry_points_reject_invalid_contracts():
    lib = bfhip.hip_lib()
    e = _err()
    s = C.c_void_p(1)
    good = dict(batches=1, cameras=6, depth_bins=118, height=32, width=88, channels=80,
                minimum=(-54, -54, -10), step=(0.3, 0.3, 20), cells=(360, 360, 1))

    def desc(**kw):
        a = {**good, **kw}
        return bfhip.lss_desc(a["batches"], a["cameras"], a["depth_bins"], a["height"],
                              a["width"], a["channels"], a["minimum"], a["step"], a["cells"])

    plan = C.c_void_p()
    assert lib.bf_cuda_lss_plan_create(None, C.byref(plan), e, 256) == 0
    assert b"invalid" in e.value and not plan
    bad = [desc(depth_bins=0), desc(depth_bins=129), desc(channels=0),
           desc(step=(0.3, 0.0, 20)), desc(step=(0.3, -1.0, 20)),
           desc(step=(float("inf"), 0.3, 20)), desc(minimum=(float("nan"), 0, 0)),
           desc(cells=(360, 0, 1)), desc(cells=(1 << 31, 1, 1))]
    for d in bad:
        e.value = b""
        assert lib.bf_cuda_lss_plan_create(C.byref(d), C.byref(plan), e, 256) == 0
        assert b"invalid" in e.value and not plan
        assert lib.bf_cuda_lss_lift_pool_f32(s, s, s, s, C.byref(d), None, e, 256) == 0
        assert lib.bf_cuda_lss_geometry_to_ranks_f32(s, s, C.byref(d), None, e, 256) == 0
        assert lib.bf_cuda_lss_lift_pool_ranks_f32(s, s, s, s, C.byref(d), None, e, 256) == 0
    # valid contract whose element counts overflow 32-bit indexing
    huge = desc(cells=(50000, 50000, 1))
    assert lib.bf_cuda_lss_plan_create(C.byref(huge), C.byref(plan), e, 256) == 0
    assert b"overflow" in e.value
    assert lib.bf_cuda_lss_lift_pool_f32(s, s, s, s, C.byref(huge), None, e, 256) == 0
    assert b"overflow" in e.value
    d = desc()
    assert lib.bf_cuda_lss_lift_pool_f32(None, s, s, s, C.byref(d), None, e, 256) == 0
    assert lib.bf_cuda_lss_lift_pool_ranks_f32(s, s, None, s, C.byref(d), None, e, 256) == 0
    assert lib.bf_cuda_lss_geometry_to_ranks_f32(s, None, C.byref(d), None, e, 256) == 0
    assert lib.bf_cuda_lss_plan_prepare_geometry_f32(None, s, None, e, 256) == 0
    assert lib.bf_cuda_lss_plan_prepare_calibration_f32(None, s, s, s, s, s, s, None, None,
                                                        None, e, 256) == 0
    e.value = b""
    assert lib.bf_cuda_lss_plan_forward_f32(None, s, s, s, None, e, 256) == 0
    assert b"unprepared" in e.value
    assert lib.bf_cuda_lss_plan_resident_bytes(None) == 0
    lib.bf_cuda_lss_plan_destroy(None)


def test_bev_stage_rejects_invalid_contracts(tmp_path):
    from bfhip import bfw
    lib = bfhip.hip_lib()
    e = _err()
    s = C.c_void_p(1)
    out = C.c_void_p()
    path = bfw.write_bev_stage(tmp_path / "bev.bfw", seed=0)
    with bfhip.Model(path) as m:
        for h, w in ((0, 8), (8, 0), (7, 8), (8, 9)):
            e.value = b""
            assert lib.bf_cuda_bev_stage_create(m.handle, h, w, C.byref(out), e, 256) == 0
            assert b"invalid" in e.value and not out
        assert lib.bf_cuda_bev_stage_create(None, 8, 8, C.byref(out), e, 256) == 0
        assert lib.bf_cuda_bev_stage_create(m.handle, 8, 8, None, e, 256) == 0
        assert lib.bf_cuda_bev_stage_create(m.handle, 1 << 20, 1 << 20, C.byref(out), e, 256) == 0
        assert b"too large" in e.value
    e.value = b""
    assert lib.bf_cuda_bev_stage_forward(None, s, s, s, s, None, e, 256) == 0
    assert b"invalid" in e.value
    assert lib.bf_cuda_bev_stage_resident_bytes(None) == 0
    lib.bf_cuda_bev_stage_destroy(None)


def test_transfusion_rejects_invalid_contracts(tmp_path):
    from bfhip import bfw
    lib = bfhip.hip_lib()
    e = _err()
    s = C.c_void_p(1)
    out = C.c_void_p()
    path = bfw.write_transfusion(tmp_path / "tf.bfw", seed=0)
    with bfhip.Model(path) as m:
        for h, w, p in ((0, 8, 10), (8, 0, 10), (8, 8, 0), (8, 8, 201), (1 << 17, 1 << 16, 10)):
            e.value = b""
            assert lib.bf_cuda_transfusion_create(m.handle, h, w, p, C.byref(out), e, 256) == 0
            assert b"invalid" in e.value and not out
        # Fewer candidates (10 * H * W) than proposals.
        assert lib.bf_cuda_transfusion_create(m.handle, 2, 2, 41, C.byref(out), e, 256) == 0
        assert b"out of range" in e.value and not out
        assert lib.bf_cuda_transfusion_create(None, 8, 8, 10, C.byref(out), e, 256) == 0
        assert lib.bf_cuda_transfusion_create(m.handle, 8, 8, 10, None, e, 256) == 0
    e.value = b""
    raw = bfhip.TfRawOutputs(*([1] * 9))
    assert lib.bf_cuda_transfusion_forward(None, s, s, C.byref(raw), None, e, 256) == 0
    assert b"invalid" in e.value
    dets = bfhip.Detections()
    assert lib.bf_cuda_transfusion_decode_detections(None, C.byref(raw), 0.1, C.byref(dets),
                                                     None, e, 256) == 0
    assert lib.bf_cuda_transfusion_resident_bytes(None) == 0
    lib.bf_cuda_transfusion_destroy(None)


def test_lidar_side_rejects_invalid_contracts(tmp_path):
    from bfhip import bfw
    lib = bfhip.hip_lib()
    e = _err()
    out = C.c_void_p()
    for args in ((0, 6, 256, 704), (10, 0, 256, 704), (1 << 33, 6, 256, 704)):
        assert lib.bf_cuda_depth_raster_create(*args, C.byref(out), e, 256) == 0 and not out
    assert lib.bf_cuda_depth_rasterize_f32(None, None, 0, None, None, None, None, None, e,
                                           256) == 0
    cfg = bfhip.voxel_config(100)
    assert lib.bf_cuda_voxelizer_create(C.byref(cfg), 0, C.byref(out), e, 256) == 0
    bad = bfhip.voxel_config(100, features=4)
    assert lib.bf_cuda_voxelizer_create(C.byref(bad), 10, C.byref(out), e, 256) == 0
    uneven = bfhip.voxel_config(100, size=(0.1234, 0.075, 0.2))
    assert lib.bf_cuda_voxelizer_create(C.byref(uneven), 10, C.byref(out), e, 256) == 0
    assert b"invalid" in e.value and not out
    assert lib.bf_cuda_voxelize_mean_f32(None, None, 0, None, None, None, None, e, 256) == 0
    path = bfw.write_lidar_backbone(tmp_path / "lidar.bfw", seed=0)
    with bfhip.Model(path) as m:
        for args in ((0, 41, 96, 96, 100), (1, 41, 96, 96, 0), (1, 2, 96, 96, 100)):
            e.value = b""
            assert lib.bf_cuda_lidar_backbone_create(m.handle, *args, C.byref(out), e, 256) == 0
            assert b"invalid" in e.value and not out
    assert lib.bf_cuda_lidar_backbone_forward(None, None, None, 0, None, None, e, 256) == 0
    assert lib.bf_cuda_lidar_backbone_forward_count_device(None, None, None, None, None, None, e,
                                                           256) == 0
    for fn in ("depth_raster", "voxelizer", "lidar_backbone"):
        assert getattr(lib, f"bf_cuda_{fn}_resident_bytes")(None) == 0
        getattr(lib, f"bf_cuda_{fn}_destroy")(None)


def test_runtime_rejects_invalid_contracts(tmp_path):
    lib = bfhip.hip_lib()
    e = _err()
    out = C.c_void_p()
    missing = str(tmp_path / "missing.bfw").encode()
    for args in ((None, 10, 10, 10), (missing, 0, 10, 10), (missing, 10, 0, 10),
                 (missing, 10, 20, 10)):
        e.value = b""
        assert lib.bf_cuda_runtime_create(*args, C.byref(out), e, 256) == 0 and not out
        assert e.value
    assert lib.bf_cuda_runtime_infer(None, None, None, e, 256) == 0
    assert lib.bf_cuda_runtime_debug_bev_stats(None, None, e, 256) == 0
    assert lib.bf_cuda_runtime_debug_hashes(None, None, e, 256) == 0
    assert lib.bf_cuda_runtime_resident_bytes(None) == 0
    lib.bf_cuda_runtime_destroy(None)
    m = bfhip.model_lib()
    assert m.bf_frame_open(missing, C.byref(out), e, 256) == 0 and not out
    assert m.bf_frame_input_view(None) is not None and not m.bf_frame_input_view(None)
    assert m.bf_frame_file_bytes(None) == 0
    m.bf_frame_close(None)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")
@pytest.mark.parametrize("order", ["sparse_first", "operators_first", "sparse_only"])
def test_sparse_types_header_coexists_with_operator_header(tmp_path, order):
    """include/bf_sparse_types.h carries only the two sparse types of the
    reference's CPU operator header (include/bf_kernels.h:34-46).  With a
    header of that name and guard on the include path (a stand-in declaring
    the types and one operator), a translation unit that includes both in
    either order must compile and still see the operator declaration; with
    none on the path the types come from bf_sparse_types.h alone."""
    ops = tmp_path / "ops"
    ops.mkdir()
    (ops / "bf_kernels.h").write_text(
        "#ifndef BF_KERNELS_H\n#define BF_KERNELS_H\n#include <stddef.h>\n#include <stdint.h>\n"
        "typedef struct { int32_t batch, z, y, x; } bf_coord4;\n"
        "typedef struct { size_t batches; int submanifold; } bf_sparse_conv3d_desc;\n"
        "int operator_marker(const bf_coord4 *c);\n#endif\n")
    lines = {"sparse_first": ['#include "bf_cuda_lidar.h"', '#include "bf_kernels.h"'],
             "operators_first": ['#include "bf_kernels.h"', '#include "bf_cuda_lidar.h"'],
             "sparse_only": ['#include "bf_cuda_lidar.h"', '#include "bf_voxel.h"',
                             '#include "bf_cuda_voxel.h"']}[order]
    use = ("int f(const bf_coord4 *c) { return operator_marker(c); }\n" if order != "sparse_only"
           else "int f(const bf_coord4 *c, const bf_sparse_conv3d_desc *d) "
                "{ return c->x + (int)d->pad_width; }\n")
    src = tmp_path / "tu.c"
    src.write_text("\n".join(lines) + "\n" + use)
    inc = [f"-I{ROOT / 'include'}"] + ([f"-I{ops}"] if order != "sparse_only" else [])
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-c", str(src), "-o",
                        str(tmp_path / "tu.o"), *inc], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
