"""Python host side of the gfx950 camera-path library.

Thin ctypes mirror of the C ABI in ``include/bf_cuda_ops.h``,
``include/bf_cuda_swin.h``, ``include/bf_cuda_camera.h``, ``include/bf_cuda.h``,
``include/bf_cuda_bev.h`` and ``include/bf_cuda_transfusion.h`` (the
reference's operator/plugin interface for this path, the lift-splat pooling
that consumes it, the BEV stage after it and the TransFusion decoder).  PyTorch supplies device memory and
the current HIP stream; every computation runs in ``lib/libbfhip.so``.  There
is no fallback: if the library is missing, importing an entry point raises.
"""

from __future__ import annotations

import ctypes as C
import pathlib

PKG = pathlib.Path(__file__).resolve().parent.parent
LIB_DIR = PKG / "lib"
HIP_LIB = LIB_DIR / "libbfhip.so"
MODEL_LIB = LIB_DIR / "libbfmodel.so"

_vp, _sz, _i = C.c_void_p, C.c_size_t, C.c_int


class BfHipError(RuntimeError):
    pass


class ConvDesc(C.Structure):
    """``bf_cuda_conv2d_desc`` (include/bf_cuda_ops.h)."""
    _fields_ = [(n, C.c_int) for n in (
        "batches", "input_channels", "output_channels", "input_height", "input_width",
        "kernel_height", "kernel_width", "stride_height", "stride_width", "padding_height",
        "padding_width", "output_height", "output_width", "transpose", "relu")]


class LssDesc(C.Structure):
    """``bf_lss_desc`` (include/bf_lss.h)."""
    _fields_ = [("batches", _sz), ("cameras", _sz), ("depth_bins", _sz),
                ("feature_height", _sz), ("feature_width", _sz), ("channels", _sz),
                ("grid_minimum", C.c_float * 3), ("grid_step", C.c_float * 3),
                ("grid_cells", _sz * 3)]


def lss_desc(batches, cameras, depth_bins, height, width, channels, minimum, step, cells):
    return LssDesc(batches, cameras, depth_bins, height, width, channels,
                   (C.c_float * 3)(*minimum), (C.c_float * 3)(*step), (_sz * 3)(*cells))


_lssp = C.POINTER(LssDesc)


class TfRawOutputs(C.Structure):
    """``bf_transfusion_raw_outputs`` (include/bf_transfusion_decoder.h)."""
    _fields_ = [(n, _vp) for n in (
        "center", "height", "dimension_log", "rotation", "velocity", "heatmap_logits",
        "query_scores", "labels", "indices")]


class Detection(C.Structure):
    """``bf_detection`` (include/bevfusion.h)."""
    _fields_ = [(n, C.c_float) for n in ("x", "y", "z", "width", "length", "height", "yaw",
                                         "velocity_x", "velocity_y", "score")] + \
               [("class_id", C.c_int)]


class Detections(C.Structure):
    """``bf_detections`` (include/bevfusion.h): BF_MAX_PROPOSALS items + count."""
    _fields_ = [("items", Detection * 200), ("count", C.c_int)]


_tfp = C.POINTER(TfRawOutputs)


class VoxelConfig(C.Structure):
    """``bf_voxel_config`` (include/bf_voxel.h)."""
    _fields_ = [("minimum", C.c_float * 3), ("maximum", C.c_float * 3),
                ("voxel_size", C.c_float * 3), ("point_features", _sz),
                ("max_points_per_voxel", _sz), ("max_voxels", _sz)]


class FrameInput(C.Structure):
    """``bf_frame_input`` (include/bf_runtime.h)."""
    _fields_ = [("camera_images", C.c_void_p), ("points", C.c_void_p), ("point_count", C.c_size_t),
                ("camera_intrinsics_6x16", C.c_void_p), ("camera_to_lidar_6x16", C.c_void_p),
                ("image_augmentation_6x16", C.c_void_p), ("lidar_augmentation_16", C.c_void_p),
                ("lidar_to_image_6x16", C.c_void_p)]


FRAME_KEYS = ("images", "points", "camera_intrinsics", "camera_to_lidar", "image_augmentation",
              "lidar_augmentation", "lidar_to_image")


def frame_input(frame):
    """A FrameInput over a dict of host float32 arrays (frame_scene.frame
    layout); returns (FrameInput, arrays kept alive by the caller)."""
    import numpy as np
    arrs = {k: np.ascontiguousarray(frame[k], np.float32) for k in FRAME_KEYS}
    ptr = lambda k: arrs[k].ctypes.data
    fi = FrameInput(ptr("images"), ptr("points"), arrs["points"].shape[0],
                    ptr("camera_intrinsics"), ptr("camera_to_lidar"), ptr("image_augmentation"),
                    ptr("lidar_augmentation"), ptr("lidar_to_image"))
    return fi, arrs


def voxel_config(max_voxels, minimum=(-54.0, -54.0, -5.0), maximum=(54.0, 54.0, 3.0),
                 size=(0.075, 0.075, 0.2), features=5, max_points=10):
    """The reference runtime's voxel contract (runtime.c:262-265) by default."""
    return VoxelConfig((C.c_float * 3)(*minimum), (C.c_float * 3)(*maximum),
                       (C.c_float * 3)(*size), features, max_points, max_voxels)

# Every symbol declared by include/*.h, with its ctypes signature.
SIGNATURES = {
    "bf_cuda_conv2d_f32": (_i, [C.POINTER(ConvDesc), _vp, _vp, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bf_cuda_gemm_f32": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, C.c_char_p, _sz]),
    "bf_cuda_swin_create": (_i, [_vp, _sz, _sz, _sz, C.POINTER(_vp), C.c_char_p, _sz]),
    "bf_cuda_swin_destroy": (None, [_vp]),
    "bf_cuda_swin_resident_bytes": (_sz, [_vp]),
    "bf_cuda_swin_forward": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bf_cuda_camera_neck_create": (_i, [_vp, _sz, _sz, _sz, _sz, _sz, C.POINTER(_vp),
                                        C.c_char_p, _sz]),
    "bf_cuda_camera_neck_destroy": (None, [_vp]),
    "bf_cuda_camera_neck_resident_bytes": (_sz, [_vp]),
    "bf_cuda_camera_fpn_forward": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bf_cuda_camera_depth_forward": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bf_cuda_camera_neck_forward": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                         C.c_char_p, _sz]),
    "bf_cuda_camera_downsample_forward": (_i, [_vp, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bfhip_swin_profile_op": (_i, [_vp, _i, _i, _i, _vp, C.c_char_p, _sz]),
    "bfhip_swin_profile_io": (_i, [_vp, _i, _i, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bfhip_camera_profile_pack": (_i, [_vp, _vp, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bfhip_camera_profile_layer": (_i, [_vp, _i, _vp, C.c_char_p, _sz]),
    "bfhip_camera_profile_layer_io": (_i, [_vp, _i, _vp, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bfhip_calibrate": (_i, [_i, _i, _i, _vp, _vp, _sz, _vp, C.c_char_p, _sz]),
    "bfhip_debug_runtime_fail_next": (_i, [_vp, C.c_char_p, _sz]),
    "bfhip_debug_camera_gather": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bfhip_debug_fpn_upsample": (_i, [_vp, _i, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bfhip_debug_swin_merge_gather": (_i, [_vp, _i, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bfhip_debug_window_map": (_i, [_i, _i, _i, _i, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bfhip_debug_window_attention": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp,
                                          C.c_char_p, _sz]),
    "bfhip_debug_window_attention_noalloc": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i,
                                                  _vp, C.c_char_p, _sz]),
    "bf_cuda_available": (_i, [C.c_char_p, _sz]),
    "bf_cuda_lss_lift_pool_f32": (_i, [_vp, _vp, _vp, _vp, _lssp, _vp, C.c_char_p, _sz]),
    "bf_cuda_lss_geometry_to_ranks_f32": (_i, [_vp, _vp, _lssp, _vp, C.c_char_p, _sz]),
    "bf_cuda_lss_lift_pool_ranks_f32": (_i, [_vp, _vp, _vp, _vp, _lssp, _vp, C.c_char_p, _sz]),
    "bf_cuda_lss_plan_create": (_i, [_lssp, C.POINTER(_vp), C.c_char_p, _sz]),
    "bf_cuda_lss_plan_destroy": (None, [_vp]),
    "bf_cuda_lss_plan_resident_bytes": (_sz, [_vp]),
    "bf_cuda_lss_plan_prepare_geometry_f32": (_i, [_vp, _vp, _vp, C.c_char_p, _sz]),
    "bf_cuda_lss_plan_prepare_calibration_f32": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                                      _vp, _vp, C.c_char_p, _sz]),
    "bf_cuda_lss_plan_forward_f32": (_i, [_vp, _vp, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bf_cuda_bev_stage_create": (_i, [_vp, _sz, _sz, C.POINTER(_vp), C.c_char_p, _sz]),
    "bf_cuda_bev_stage_destroy": (None, [_vp]),
    "bf_cuda_bev_stage_forward": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bf_cuda_bev_stage_resident_bytes": (_sz, [_vp]),
    "bf_cuda_transfusion_create": (_i, [_vp, _sz, _sz, _sz, C.POINTER(_vp), C.c_char_p, _sz]),
    "bf_cuda_transfusion_destroy": (None, [_vp]),
    "bf_cuda_transfusion_forward": (_i, [_vp, _vp, _vp, _tfp, _vp, C.c_char_p, _sz]),
    "bf_cuda_transfusion_decode_detections": (_i, [_vp, _tfp, C.c_float, C.POINTER(Detections),
                                                   _vp, C.c_char_p, _sz]),
    "bf_cuda_transfusion_resident_bytes": (_sz, [_vp]),
    "bf_cuda_depth_raster_create": (_i, [_sz, _sz, _sz, _sz, C.POINTER(_vp), C.c_char_p, _sz]),
    "bf_cuda_depth_raster_destroy": (None, [_vp]),
    "bf_cuda_depth_raster_resident_bytes": (_sz, [_vp]),
    "bf_cuda_depth_rasterize_f32": (_i, [_vp, _vp, _sz, _vp, _vp, _vp, _vp, _vp, C.c_char_p,
                                         _sz]),
    "bf_cuda_voxelizer_create": (_i, [C.POINTER(VoxelConfig), _sz, C.POINTER(_vp), C.c_char_p,
                                      _sz]),
    "bf_cuda_voxelizer_destroy": (None, [_vp]),
    "bf_cuda_voxelizer_resident_bytes": (_sz, [_vp]),
    "bf_cuda_voxelize_mean_f32": (_i, [_vp, _vp, _sz, _vp, _vp, _vp, _vp, C.c_char_p, _sz]),
    "bf_cuda_lidar_backbone_create": (_i, [_vp, _sz, _sz, _sz, _sz, _sz, C.POINTER(_vp),
                                           C.c_char_p, _sz]),
    "bf_cuda_lidar_backbone_destroy": (None, [_vp]),
    "bf_cuda_lidar_backbone_resident_bytes": (_sz, [_vp]),
    "bf_cuda_lidar_backbone_forward": (_i, [_vp, _vp, _vp, _sz, _vp, _vp, C.c_char_p, _sz]),
    "bf_cuda_lidar_backbone_forward_count_device": (_i, [_vp, _vp, _vp, _vp, _vp, _vp,
                                                         C.c_char_p, _sz]),
    "bf_cuda_runtime_create": (_i, [C.c_char_p, _sz, _sz, _sz, C.POINTER(_vp), C.c_char_p, _sz]),
    "bf_cuda_runtime_destroy": (None, [_vp]),
    "bf_cuda_runtime_infer": (_i, [_vp, C.POINTER(FrameInput), C.POINTER(Detections),
                                   C.c_char_p, _sz]),
    "bf_cuda_runtime_resident_bytes": (_sz, [_vp]),
    "bf_cuda_runtime_debug_bev_stats": (_i, [_vp, C.POINTER(C.c_float), C.c_char_p, _sz]),
    "bf_cuda_runtime_debug_hashes": (_i, [_vp, C.POINTER(C.c_ulonglong), C.c_char_p, _sz]),
}

SWIN_OPS = ("ln1", "qkv", "attention", "proj", "ln2", "fc1", "fc2", "merge", "mlp", "wmsa")

MODEL_SIGNATURES = {
    "bf_model_open": (_i, [C.c_char_p, C.POINTER(_vp), C.c_char_p, _sz]),
    "bf_model_close": (None, [_vp]),
    "bf_model_tensor_count": (_sz, [_vp]),
    "bf_model_file_bytes": (C.c_uint64, [_vp]),
    "bf_model_tensor_at": (_vp, [_vp, _sz]),
    "bf_model_find": (_vp, [_vp, C.c_char_p]),
    "bf_model_validate_tensor": (_i, [_vp, _vp, C.c_char_p, _sz]),
    "bf_model_validate_all": (_i, [_vp, C.c_char_p, _sz]),
    "bf_dtype_name": (C.c_char_p, [C.c_uint32]),
    "bf_frame_open": (_i, [C.c_char_p, C.POINTER(_vp), C.c_char_p, _sz]),
    "bf_frame_close": (None, [_vp]),
    "bf_frame_input_view": (C.POINTER(FrameInput), [_vp]),
    "bf_frame_file_bytes": (_sz, [_vp]),
}

_model_lib = None
_hip_lib = None


def _bind(lib, table):
    """Attach signatures; a symbol the library lacks raises when first used."""
    for name, (res, args) in table.items():
        if hasattr(lib, name):
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
    return lib


def missing_symbols():
    """Entry points declared in include/*.h that libbfhip.so does not export."""
    lib = hip_lib()
    return [n for n in SIGNATURES if not hasattr(lib, n)]


def model_lib():
    global _model_lib
    if _model_lib is None:
        if not MODEL_LIB.exists():
            raise BfHipError(f"{MODEL_LIB} is not built (run __graft_entry__.build())")
        _model_lib = _bind(C.CDLL(str(MODEL_LIB), mode=C.RTLD_GLOBAL), MODEL_SIGNATURES)
    return _model_lib


def hip_lib():
    """Load libbfhip.so; raises BfHipError if it is missing (no CPU fallback)."""
    global _hip_lib
    if _hip_lib is None:
        model_lib()
        if not HIP_LIB.exists():
            raise BfHipError(f"{HIP_LIB} is not built (run __graft_entry__.build())")
        _hip_lib = _bind(C.CDLL(str(HIP_LIB)), SIGNATURES)
    return _hip_lib


def _err():
    return C.create_string_buffer(512)


def _check(ok, err, what):
    if not ok:
        raise BfHipError(f"{what}: {err.value.decode(errors='replace')}")


class Model:
    """A BFW container opened through libbfmodel.so."""

    def __init__(self, path):
        lib = model_lib()
        self.handle, err = _vp(), _err()
        _check(lib.bf_model_open(str(path).encode(), C.byref(self.handle), err, 512), err,
               f"open {path}")

    def close(self):
        if self.handle:
            model_lib().bf_model_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------- torch glue
def _torch():
    import torch
    return torch


def _ptr(t):
    if t is None:
        return None
    torch = _torch()
    if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous():
        raise BfHipError("expected a contiguous float32 device tensor")
    return _vp(t.data_ptr())


def _iptr(t):
    torch = _torch()
    if not t.is_cuda or t.dtype != torch.int32 or not t.is_contiguous():
        raise BfHipError("expected a contiguous int32 device tensor")
    return _vp(t.data_ptr())


def _stream(stream=None):
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return _vp(s.cuda_stream)


def gemm_f32(x, w, b=None, relu=False, out=None, stream=None):
    """out[M,N] = x[M,K] @ w[N,K]^T + b (bf_cuda_gemm_f32)."""
    torch = _torch()
    M, K = x.shape
    N = w.shape[0]
    out = out if out is not None else torch.empty((M, N), device=x.device, dtype=torch.float32)
    err = _err()
    _check(hip_lib().bf_cuda_gemm_f32(_ptr(x), _ptr(w), _ptr(b), _ptr(out), M, K, N, int(relu),
                                      _stream(stream), err, 512), err, "bf_cuda_gemm_f32")
    return out


CALIB_KINDS = ("empty", "mfma16", "mfma32", "lds", "copy", "mfma_lds", "mfma_lds_flat",
               "mfma_lds_narrow", "mfma_lds_narrow_flat")


def calibrate(kind, grid, iters=0, src=None, dst=None, stream=None):
    """Enqueue one calibration kernel (include/bfhip_profile.h): `kind` in
    CALIB_KINDS; `dst` (and `src` for "copy") are device tensors."""
    err = _err()
    nbytes = dst.numel() * dst.element_size() if dst is not None else 0
    _check(hip_lib().bfhip_calibrate(CALIB_KINDS.index(kind), grid, iters,
                                     _vp(src.data_ptr()) if src is not None else None,
                                     _vp(dst.data_ptr()) if dst is not None else None,
                                     nbytes, _stream(stream), err, 512),
           err, "bfhip_calibrate")


def conv_desc(x_shape, w_shape, stride=(1, 1), padding=(0, 0), transpose=False, relu=False,
              out_hw=None, output_channels=None):
    n, ci, ih, iw = x_shape
    if transpose:
        co = output_channels or w_shape[1]
        kh, kw = w_shape[2], w_shape[3]
        oh = (ih - 1) * stride[0] - 2 * padding[0] + kh
        ow = (iw - 1) * stride[1] - 2 * padding[1] + kw
    else:
        co, kh, kw = w_shape[0], w_shape[2], w_shape[3]
        oh = (ih + 2 * padding[0] - kh) // stride[0] + 1
        ow = (iw + 2 * padding[1] - kw) // stride[1] + 1
    if out_hw is not None:
        oh, ow = out_hw
    return ConvDesc(n, ci, co, ih, iw, kh, kw, stride[0], stride[1], padding[0], padding[1],
                    oh, ow, int(transpose), int(relu))


def conv2d_f32(x, w, b=None, stride=(1, 1), padding=(0, 0), transpose=False, relu=False,
               out_hw=None, out=None, stream=None):
    """NCHW convolution (bf_cuda_conv2d_f32); weights OIHW or IOHW if transpose."""
    torch = _torch()
    d = conv_desc(tuple(x.shape), tuple(w.shape), stride, padding, transpose, relu, out_hw)
    shape = (d.batches, d.output_channels, d.output_height, d.output_width)
    out = out if out is not None else torch.empty(shape, device=x.device, dtype=torch.float32)
    err = _err()
    _check(hip_lib().bf_cuda_conv2d_f32(C.byref(d), _ptr(x), _ptr(w), _ptr(b), _ptr(out),
                                        _stream(stream), err, 512), err, "bf_cuda_conv2d_f32")
    return out


def conv2d_raw(desc, x, w, b, out, stream=None):
    """Call bf_cuda_conv2d_f32 with an explicit descriptor; returns (ok, message)."""
    err = _err()
    ok = hip_lib().bf_cuda_conv2d_f32(C.byref(desc), x, w, b, out, _stream(stream), err, 512)
    return bool(ok), err.value.decode(errors="replace")


def window_map(batches, height, width, shift, device, stream=None):
    """Device window partition (include/bfhip_debug.h): (token, label) int32."""
    torch = _torch()
    n = batches * (-(-height // 7)) * (-(-width // 7)) * 49
    token = torch.empty(n, dtype=torch.int32, device=device)
    label = torch.empty(n, dtype=torch.int32, device=device)
    err = _err()
    _check(hip_lib().bfhip_debug_window_map(batches, height, width, shift,
                                            _vp(token.data_ptr()), _vp(label.data_ptr()),
                                            _stream(stream), err, 512), err,
           "bfhip_debug_window_map")
    return token, label


def window_attention(qkv, qkv_bias, bias_mat, batches, height, width, heads, shift, out=None,
                     stream=None, noalloc=False):
    """Production window-attention kernel on caller buffers (include/bfhip_debug.h):
    qkv fp16 [tokens, 96*heads], qkv_bias fp32 [96*heads], bias_mat fp32
    [heads, 49, 49]; returns out fp16 [tokens, 32*heads].  noalloc selects
    bfhip_debug_window_attention_noalloc (score terms in the library's static
    device array; the call does not synchronise)."""
    torch = _torch()
    c = 32 * heads
    tokens = batches * height * width
    if (qkv.dtype != torch.float16 or tuple(qkv.shape) != (tokens, 3 * c)
            or not qkv.is_contiguous()):
        raise BfHipError("qkv must be a contiguous fp16 [tokens, 3C] tensor")
    if tuple(qkv_bias.shape) != (3 * c,) or tuple(bias_mat.shape) != (heads, 49, 49):
        raise BfHipError("qkv_bias must be [3C] and bias_mat [heads, 49, 49]")
    out = out if out is not None else torch.zeros((tokens, c), dtype=torch.float16,
                                                  device=qkv.device)
    err = _err()
    name = "bfhip_debug_window_attention_noalloc" if noalloc else "bfhip_debug_window_attention"
    _check(getattr(hip_lib(), name)(
        _vp(qkv.data_ptr()), _ptr(qkv_bias), _ptr(bias_mat), _vp(out.data_ptr()), batches,
        height, width, c, heads, shift, _stream(stream), err, 512), err, name)
    return out


def camera_gather(neck, layer, src0, src1=None, affine=None, stream=None):
    """A-operand gather of camera-neck conv `layer` over identity weights
    (bfhip_debug_camera_gather, include/bfhip_debug.h): returns fp32 [M, K],
    the gathered operand of the production loader instance."""
    torch = _torch()
    layers = {1: (3, 1, 1), 3: (3, 1, 1), 4: (5, 4, 2), 5: (5, 2, 2), 6: (3, 1, 1),
              7: (3, 1, 1), 8: (1, 1, 0), 9: (3, 1, 1), 10: (3, 2, 1), 11: (3, 1, 1)}
    if layer not in layers:
        raise BfHipError(f"no gather probe for camera layer {layer}")
    k, st, pad = layers[layer]
    if layer == 4:
        if src0.dtype != torch.float32 or src0.dim() != 3 or affine is None:
            raise BfHipError("dtransform.3 takes fp32 depth [B, H, W] and a 16-float affine")
        n, ih, iw = src0.shape
        ci = 8
    else:
        if src0.dtype != torch.float16 or src0.dim() != 4:
            raise BfHipError("src0 must be fp16 [B, H, W, C]")
        n, ih, iw, ci = src0.shape
        if layer == 6:
            if src1 is None or src1.dtype != torch.float16 or tuple(src1.shape[:3]) != (n, ih, iw):
                raise BfHipError("depthnet.0 takes src1 fp16 [B, H, W, 256]")
            ci += src1.shape[3]
    for t in (src0, src1, affine):
        if t is not None and not t.is_contiguous():
            raise BfHipError("probe inputs must be contiguous")
    oh, ow = (ih + 2 * pad - k) // st + 1, (iw + 2 * pad - k) // st + 1
    out = torch.empty((n * oh * ow, k * k * ci), dtype=torch.float32, device=src0.device)
    err = _err()
    _check(hip_lib().bfhip_debug_camera_gather(
        neck.handle, layer, _vp(src0.data_ptr()), _vp(src1.data_ptr() if src1 is not None else None),
        _vp(affine.data_ptr() if affine is not None else None), _vp(out.data_ptr()),
        _stream(stream), err, 512), err, "bfhip_debug_camera_gather")
    return out


def fpn_upsample(neck, level, up, stream=None):
    """Lateral-conv epilogue over a zero product (bfhip_debug_fpn_upsample):
    up fp32 [B, h, w, 256] -> fp16 [B, H, W, 256] = fp16(relu(bilinear(up)))."""
    torch = _torch()
    if up.dtype != torch.float32 or up.dim() != 4 or up.shape[3] != 256 or not up.is_contiguous():
        raise BfHipError("up must be a contiguous fp32 [B, h, w, 256] tensor")
    big = (neck.h, neck.w)
    mid = (-(-neck.h // 2), -(-neck.w // 2))
    H, W = big if level == 0 else mid
    out = torch.empty((up.shape[0], H, W, 256), dtype=torch.float16, device=up.device)
    err = _err()
    _check(hip_lib().bfhip_debug_fpn_upsample(neck.handle, level, _ptr(up), _vp(out.data_ptr()),
                                              _stream(stream), err, 512),
           err, "bfhip_debug_fpn_upsample")
    return out


def swin_merge_gather(swin, stage, xh, stream=None):
    """Patch-merge gather of stage `stage` over permuted identity weights
    (bfhip_debug_swin_merge_gather): xh fp16 [B, H, W, C] -> fp32
    [B*H2*W2, 4C] in the reference's unfold column order."""
    torch = _torch()
    if xh.dtype != torch.float16 or xh.dim() != 4 or not xh.is_contiguous():
        raise BfHipError("xh must be a contiguous fp16 [B, H, W, C] tensor")
    b, h, w, c = xh.shape
    out = torch.empty((b * -(-h // 2) * -(-w // 2), 4 * c), dtype=torch.float32, device=xh.device)
    err = _err()
    _check(hip_lib().bfhip_debug_swin_merge_gather(swin.handle, stage, _vp(xh.data_ptr()),
                                                   _vp(out.data_ptr()), _stream(stream), err, 512),
           err, "bfhip_debug_swin_merge_gather")
    return out


class Swin:
    """bf_cuda_swin context (include/bf_cuda_swin.h)."""

    def __init__(self, model: Model, batches: int, height: int, width: int):
        self.lib = hip_lib()
        self.batches, self.height, self.width = batches, height, width
        self.handle, err = _vp(), _err()
        _check(self.lib.bf_cuda_swin_create(model.handle, batches, height, width,
                                            C.byref(self.handle), err, 512), err,
               "bf_cuda_swin_create")

    def output_shapes(self):
        b, h, w = self.batches, self.height, self.width
        return [(b, c, -(-h // d), -(-w // d)) for c, d in ((192, 8), (384, 16), (768, 32))]

    def resident_bytes(self) -> int:
        return self.lib.bf_cuda_swin_resident_bytes(self.handle)

    def forward(self, images, outs=None, stream=None):
        torch = _torch()
        if outs is None:
            outs = [torch.empty(s, device=images.device, dtype=torch.float32)
                    for s in self.output_shapes()]
        err = _err()
        _check(self.lib.bf_cuda_swin_forward(self.handle, _ptr(images), *map(_ptr, outs),
                                             _stream(stream), err, 512), err,
               "bf_cuda_swin_forward")
        return outs

    def profile_op(self, stage, block, op, stream=None):
        """Enqueue one op's kernels (include/bfhip_profile.h)."""
        err = _err()
        _check(self.lib.bfhip_swin_profile_op(self.handle, stage, block, SWIN_OPS.index(op),
                                              _stream(stream), err, 512), err,
               "bfhip_swin_profile_op")

    def profile_io(self, op, stage=0, images=None, out=None, stream=None):
        """Patch embedding ("patch_embed", reads images), the output norm of
        stage 1..3 alone ("out_norm", writes out), or the merge after stage
        1..2 with that stage's output norm in one launch ("merge_out_norm",
        writes out) on caller buffers (bfhip_swin_profile_io)."""
        err = _err()
        code = {"patch_embed": 10, "out_norm": 11, "merge_out_norm": 12}[op]
        _check(self.lib.bfhip_swin_profile_io(self.handle, stage, code,
                                              _vp(images.data_ptr() if images is not None else None),
                                              _vp(out.data_ptr() if out is not None else None),
                                              _stream(stream), err, 512), err,
               "bfhip_swin_profile_io")

    def close(self):
        if self.handle:
            self.lib.bf_cuda_swin_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class CameraNeck:
    """bf_cuda_camera_neck context (include/bf_cuda_camera.h)."""

    def __init__(self, model: Model, batches: int, feature_h: int, feature_w: int,
                 bev_h: int, bev_w: int):
        self.lib = hip_lib()
        self.batches, self.h, self.w = batches, feature_h, feature_w
        self.bev_h, self.bev_w = bev_h, bev_w
        self.handle, err = _vp(), _err()
        _check(self.lib.bf_cuda_camera_neck_create(model.handle, batches, feature_h, feature_w,
                                                   bev_h, bev_w, C.byref(self.handle), err, 512),
               err, "bf_cuda_camera_neck_create")

    def resident_bytes(self) -> int:
        return self.lib.bf_cuda_camera_neck_resident_bytes(self.handle)

    def _empty(self, shape, like):
        torch = _torch()
        return torch.empty(shape, device=like.device, dtype=torch.float32)

    def fpn_forward(self, s0, s1, s2, stream=None):
        b, h, w = self.batches, self.h, self.w
        f0 = self._empty((b, 256, h, w), s0)
        f1 = self._empty((b, 256, (h + 1) // 2, (w + 1) // 2), s0)
        err = _err()
        _check(self.lib.bf_cuda_camera_fpn_forward(self.handle, _ptr(s0), _ptr(s1), _ptr(s2),
                                                   _ptr(f0), _ptr(f1), _stream(stream), err, 512),
               err, "bf_cuda_camera_fpn_forward")
        return f0, f1

    def depth_forward(self, fpn0, depth, stream=None):
        b, h, w = self.batches, self.h, self.w
        logits = self._empty((b, 118, h, w), fpn0)
        ctx = self._empty((b, 80, h, w), fpn0)
        err = _err()
        _check(self.lib.bf_cuda_camera_depth_forward(self.handle, _ptr(fpn0), _ptr(depth),
                                                     _ptr(logits), _ptr(ctx), _stream(stream),
                                                     err, 512), err,
               "bf_cuda_camera_depth_forward")
        return logits, ctx

    def neck_forward(self, s0, s1, s2, depth, logits=None, ctx=None, stream=None):
        b, h, w = self.batches, self.h, self.w
        logits = logits if logits is not None else self._empty((b, 118, h, w), s0)
        ctx = ctx if ctx is not None else self._empty((b, 80, h, w), s0)
        err = _err()
        _check(self.lib.bf_cuda_camera_neck_forward(self.handle, _ptr(s0), _ptr(s1), _ptr(s2),
                                                    _ptr(depth), _ptr(logits), _ptr(ctx),
                                                    _stream(stream), err, 512), err,
               "bf_cuda_camera_neck_forward")
        return logits, ctx

    def downsample_forward(self, bev, out=None, stream=None):
        if out is None:
            out = self._empty((1, 80, self.bev_w // 2, self.bev_h // 2), bev)
        err = _err()
        _check(self.lib.bf_cuda_camera_downsample_forward(self.handle, _ptr(bev), _ptr(out),
                                                          _stream(stream), err, 512), err,
               "bf_cuda_camera_downsample_forward")
        return out

    def profile_layer(self, layer, stream=None):
        """Enqueue one convolution layer (include/bfhip_profile.h)."""
        err = _err()
        _check(self.lib.bfhip_camera_profile_layer(self.handle, layer, _stream(stream), err, 512),
               err, "bfhip_camera_profile_layer")

    def profile_layer_io(self, layer, inp=None, out0=None, out1=None, stream=None):
        """Enqueue dtransform.3 (layer 4, reads `inp`), depthnet.6 (layer 8,
        writes `out0` / `out1`) or the last downsample conv (layer 11, writes
        `out0`) on caller buffers (include/bfhip_profile.h)."""
        err = _err()
        _check(self.lib.bfhip_camera_profile_layer_io(self.handle, layer, _ptr(inp), _ptr(out0),
                                                      _ptr(out1), _stream(stream), err, 512),
               err, "bfhip_camera_profile_layer_io")

    def profile_pack(self, s0, s1, s2, stream=None):
        """Enqueue the pack of the three Swin levels to channels-last fp16
        (bfhip_camera_profile_pack)."""
        err = _err()
        _check(self.lib.bfhip_camera_profile_pack(self.handle, _ptr(s0), _ptr(s1), _ptr(s2),
                                                  _stream(stream), err, 512),
               err, "bfhip_camera_profile_pack")

    def close(self):
        if self.handle:
            self.lib.bf_cuda_camera_neck_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------ lift-splat pooling
def _lss_shapes(desc):
    d = desc
    return ((d.batches, d.cameras, d.depth_bins, d.feature_height, d.feature_width),
            (d.batches, d.channels * d.grid_cells[2], d.grid_cells[0], d.grid_cells[1]))


def lss_lift_pool(logits, context, geometry, desc, out=None, stream=None):
    """Stateless lift + pool with float atomics (bf_cuda_lss_lift_pool_f32)."""
    lib, err = hip_lib(), _err()
    out = out if out is not None else _torch().empty(_lss_shapes(desc)[1], device=logits.device)
    _check(lib.bf_cuda_lss_lift_pool_f32(_ptr(logits), _ptr(context), _ptr(geometry), _ptr(out),
                                         C.byref(desc), _stream(stream), err, 512),
           err, "bf_cuda_lss_lift_pool_f32")
    return out


def lss_geometry_to_ranks(geometry, desc, out=None, stream=None):
    """[B,N,D,H,W,3] -> int32 cell ranks within each batch, -1 outside."""
    lib, err = hip_lib(), _err()
    torch = _torch()
    out = out if out is not None else torch.empty(_lss_shapes(desc)[0], device=geometry.device,
                                                  dtype=torch.int32)
    _check(lib.bf_cuda_lss_geometry_to_ranks_f32(_ptr(geometry), _iptr(out), C.byref(desc),
                                                 _stream(stream), err, 512),
           err, "bf_cuda_lss_geometry_to_ranks_f32")
    return out


def lss_lift_pool_ranks(logits, context, ranks, desc, out=None, stream=None):
    """Stateless lift + pool from precomputed ranks (float atomics)."""
    lib, err = hip_lib(), _err()
    out = out if out is not None else _torch().empty(_lss_shapes(desc)[1], device=logits.device)
    _check(lib.bf_cuda_lss_lift_pool_ranks_f32(_ptr(logits), _ptr(context), _iptr(ranks),
                                               _ptr(out), C.byref(desc), _stream(stream), err,
                                               512),
           err, "bf_cuda_lss_lift_pool_ranks_f32")
    return out


class LssPlan:
    """bf_cuda_lss_plan: deterministic lift-splat pooling (include/bf_cuda.h)."""

    def __init__(self, desc: LssDesc):
        self.lib, self.desc = hip_lib(), desc
        self.handle, err = _vp(), _err()
        _check(self.lib.bf_cuda_lss_plan_create(C.byref(desc), C.byref(self.handle), err, 512),
               err, "bf_cuda_lss_plan_create")

    def resident_bytes(self) -> int:
        return self.lib.bf_cuda_lss_plan_resident_bytes(self.handle)

    def prepare_geometry(self, geometry, stream=None):
        err = _err()
        _check(self.lib.bf_cuda_lss_plan_prepare_geometry_f32(self.handle, _ptr(geometry),
                                                              _stream(stream), err, 512),
               err, "bf_cuda_lss_plan_prepare_geometry_f32")

    def prepare_calibration(self, frustum, camera_rotation, camera_translation, intrinsics,
                            post_rotation, post_translation, extra_rotation=None,
                            extra_translation=None, stream=None):
        err = _err()
        _check(self.lib.bf_cuda_lss_plan_prepare_calibration_f32(
            self.handle, _ptr(frustum), _ptr(camera_rotation), _ptr(camera_translation),
            _ptr(intrinsics), _ptr(post_rotation), _ptr(post_translation), _ptr(extra_rotation),
            _ptr(extra_translation), _stream(stream), err, 512),
            err, "bf_cuda_lss_plan_prepare_calibration_f32")

    def forward(self, logits, context, out=None, stream=None):
        out = out if out is not None else _torch().empty(_lss_shapes(self.desc)[1],
                                                         device=logits.device)
        err = _err()
        _check(self.lib.bf_cuda_lss_plan_forward_f32(self.handle, _ptr(logits), _ptr(context),
                                                     _ptr(out), _stream(stream), err, 512),
               err, "bf_cuda_lss_plan_forward_f32")
        return out

    def close(self):
        if self.handle:
            self.lib.bf_cuda_lss_plan_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# --------------------------------------------------------------- BEV stage
class BevStage:
    """bf_cuda_bev_stage context (include/bf_cuda_bev.h): batch one, H x W BEV."""

    def __init__(self, model: Model, height: int, width: int):
        self.lib, self.h, self.w = hip_lib(), height, width
        self.handle, err = _vp(), _err()
        _check(self.lib.bf_cuda_bev_stage_create(model.handle, height, width, C.byref(self.handle),
                                                 err, 512), err, "bf_cuda_bev_stage_create")

    def resident_bytes(self) -> int:
        return self.lib.bf_cuda_bev_stage_resident_bytes(self.handle)

    def forward(self, x, outs=None, stream=None):
        """x [1,336,H,W] -> (spatial [1,512,H,W], shared [1,128,H,W], heatmap [1,10,H,W])."""
        torch = _torch()
        if outs is None:
            outs = tuple(torch.empty((1, c, self.h, self.w), device=x.device)
                         for c in (512, 128, 10))
        err = _err()
        _check(self.lib.bf_cuda_bev_stage_forward(self.handle, _ptr(x), *map(_ptr, outs),
                                                  _stream(stream), err, 512),
               err, "bf_cuda_bev_stage_forward")
        return outs

    def close(self):
        if self.handle:
            self.lib.bf_cuda_bev_stage_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


TF_FIELDS = (("center", 2), ("height", 1), ("dimension_log", 3), ("rotation", 2),
             ("velocity", 2), ("heatmap_logits", 10), ("query_scores", 10))


def _lptr(t):
    torch = _torch()
    if not t.is_cuda or t.dtype != torch.int64 or not t.is_contiguous():
        raise BfHipError("expected a contiguous int64 device tensor")
    return _vp(t.data_ptr())


class TransFusion:
    """bf_cuda_transfusion context (include/bf_cuda_transfusion.h): batch one,
    H x W BEV map, `proposals` queries."""

    def __init__(self, model: Model, height: int, width: int, proposals: int = 200):
        self.lib, self.h, self.w, self.p = hip_lib(), height, width, proposals
        self.handle, err = _vp(), _err()
        _check(self.lib.bf_cuda_transfusion_create(model.handle, height, width, proposals,
                                                   C.byref(self.handle), err, 512),
               err, "bf_cuda_transfusion_create")

    def resident_bytes(self) -> int:
        return self.lib.bf_cuda_transfusion_resident_bytes(self.handle)

    def outputs(self, device):
        """Fresh raw-output tensors: channel-major [1,C,P] fp32 fields plus
        int64 labels / indices [1,P]."""
        torch = _torch()
        outs = {k: torch.empty((1, c, self.p), device=device) for k, c in TF_FIELDS}
        outs["labels"] = torch.empty((1, self.p), dtype=torch.int64, device=device)
        outs["indices"] = torch.empty((1, self.p), dtype=torch.int64, device=device)
        return outs

    @staticmethod
    def raw(outs):
        return TfRawOutputs(*[_ptr(outs[k]) for k, _ in TF_FIELDS],
                            _lptr(outs["labels"]), _lptr(outs["indices"]))

    def forward(self, shared, heatmap, outs=None, stream=None):
        """shared [1,128,H,W], heatmap logits [1,10,H,W] -> dict of raw outputs."""
        if outs is None:
            outs = self.outputs(shared.device)
        raw, err = self.raw(outs), _err()
        _check(self.lib.bf_cuda_transfusion_forward(self.handle, _ptr(shared), _ptr(heatmap),
                                                    C.byref(raw), _stream(stream), err, 512),
               err, "bf_cuda_transfusion_forward")
        return outs

    def decode(self, outs, threshold, stream=None):
        """GPU decode + range filter of one forward's outputs -> Detections
        (synchronises the stream)."""
        raw, dets, err = self.raw(outs), Detections(), _err()
        _check(self.lib.bf_cuda_transfusion_decode_detections(
            self.handle, C.byref(raw), threshold, C.byref(dets), _stream(stream), err, 512),
            err, "bf_cuda_transfusion_decode_detections")
        return dets

    def close(self):
        if self.handle:
            self.lib.bf_cuda_transfusion_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _tptr(t, dtype):
    torch = _torch()
    if not t.is_cuda or t.dtype != dtype or not t.is_contiguous():
        raise BfHipError(f"expected a contiguous {dtype} device tensor")
    return _vp(t.data_ptr())


class _Context:
    _destroy = None

    def close(self):
        if getattr(self, "handle", None):
            getattr(self.lib, self._destroy)(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DepthRaster(_Context):
    """bf_cuda_depth_raster context (include/bf_cuda_depth_raster.h)."""
    _destroy = "bf_cuda_depth_raster_destroy"

    def __init__(self, max_points, cameras=6, height=256, width=704):
        self.lib, self.shape = hip_lib(), (cameras, height, width)
        self.handle, err = _vp(), _err()
        _check(self.lib.bf_cuda_depth_raster_create(max_points, cameras, height, width,
                                                    C.byref(self.handle), err, 512),
               err, "bf_cuda_depth_raster_create")

    def resident_bytes(self):
        return self.lib.bf_cuda_depth_raster_resident_bytes(self.handle)

    def forward(self, points, lidar_aug, lidar_to_image, image_aug, out=None, stream=None):
        """points [P,5] -> dense depth [N,H,W]."""
        torch = _torch()
        if out is None:
            out = torch.empty(self.shape, device=lidar_aug.device)
        err = _err()
        pts = _ptr(points) if points.numel() else None
        _check(self.lib.bf_cuda_depth_rasterize_f32(self.handle, pts, points.shape[0],
                                                    _ptr(lidar_aug), _ptr(lidar_to_image),
                                                    _ptr(image_aug), _ptr(out), _stream(stream),
                                                    err, 512),
               err, "bf_cuda_depth_rasterize_f32")
        return out


class Voxelizer(_Context):
    """bf_cuda_voxelizer context (include/bf_cuda_voxel.h)."""
    _destroy = "bf_cuda_voxelizer_destroy"

    def __init__(self, config, max_points):
        self.lib, self.config = hip_lib(), config
        self.handle, err = _vp(), _err()
        _check(self.lib.bf_cuda_voxelizer_create(C.byref(config), max_points,
                                                 C.byref(self.handle), err, 512),
               err, "bf_cuda_voxelizer_create")

    def resident_bytes(self):
        return self.lib.bf_cuda_voxelizer_resident_bytes(self.handle)

    def forward(self, points, coords=None, means=None, count=None, stream=None):
        """points [P,5] -> (coords int32 [max_voxels,4], means [max_voxels,5],
        count int32 [1]); rows below count are valid."""
        torch = _torch()
        v, dev = self.config.max_voxels, points.device
        coords = coords if coords is not None else torch.empty((v, 4), dtype=torch.int32, device=dev)
        means = means if means is not None else torch.empty((v, 5), device=dev)
        count = count if count is not None else torch.empty((1,), dtype=torch.int32, device=dev)
        err = _err()
        _check(self.lib.bf_cuda_voxelize_mean_f32(
            self.handle, _ptr(points) if points.numel() else None, points.shape[0],
            _tptr(coords, torch.int32), _ptr(means), _tptr(count, torch.int32), _stream(stream),
            err, 512), err, "bf_cuda_voxelize_mean_f32")
        return coords, means, count


class LidarBackbone(_Context):
    """bf_cuda_lidar_backbone context (include/bf_cuda_lidar.h)."""
    _destroy = "bf_cuda_lidar_backbone_destroy"

    def __init__(self, model: Model, batches, depth, height, width, capacity):
        self.lib = hip_lib()
        d, h, w = depth, height, width
        for pz in (1, 1, 0):
            d, h, w = (d + 2 * pz - 3) // 2 + 1, (h - 1) // 2 + 1, (w - 1) // 2 + 1
        self.out_shape = (batches, 128, (d - 3) // 2 + 1, h, w)
        self.handle, err = _vp(), _err()
        _check(self.lib.bf_cuda_lidar_backbone_create(model.handle, batches, depth, height, width,
                                                      capacity, C.byref(self.handle), err, 512),
               err, "bf_cuda_lidar_backbone_create")

    def resident_bytes(self):
        return self.lib.bf_cuda_lidar_backbone_resident_bytes(self.handle)

    def forward(self, coords, features, count, out=None, stream=None):
        """coords int32 [N,4], MeanVFE features [N,5]; count an int or a
        device int32 [1] tensor -> dense [B,128,D',H',W']."""
        torch = _torch()
        if out is None:
            out = torch.empty(self.out_shape, device=features.device)
        err = _err()
        if isinstance(count, int):
            ok = self.lib.bf_cuda_lidar_backbone_forward(
                self.handle, _tptr(coords, torch.int32), _ptr(features), count, _ptr(out),
                _stream(stream), err, 512)
        else:
            ok = self.lib.bf_cuda_lidar_backbone_forward_count_device(
                self.handle, _tptr(coords, torch.int32), _ptr(features), _tptr(count, torch.int32),
                _ptr(out), _stream(stream), err, 512)
        _check(ok, err, "bf_cuda_lidar_backbone_forward")
        return out


class FrameFile(_Context):
    """A BFI frame mapped by libbfmodel.so (include/bf_frame.h)."""
    _destroy = "bf_frame_close"

    def __init__(self, path):
        self.lib = model_lib()
        self.handle, err = _vp(), _err()
        _check(self.lib.bf_frame_open(str(path).encode(), C.byref(self.handle), err, 512), err,
               "bf_frame_open")

    @property
    def input(self) -> FrameInput:
        return self.lib.bf_frame_input_view(self.handle).contents

    def bytes(self):
        return self.lib.bf_frame_file_bytes(self.handle)


class Runtime(_Context):
    """bf_cuda_runtime (include/bf_cuda_runtime.h): BFW checkpoint in, host
    frame in, canonical detections out."""
    _destroy = "bf_cuda_runtime_destroy"

    def __init__(self, model_path, point_capacity=300000, voxel_capacity=160000,
                 sparse_capacity=160000):
        self.lib = hip_lib()
        self.handle, err = _vp(), _err()
        _check(self.lib.bf_cuda_runtime_create(str(model_path).encode(), point_capacity,
                                               voxel_capacity, sparse_capacity,
                                               C.byref(self.handle), err, 512),
               err, "bf_cuda_runtime_create")

    def resident_bytes(self):
        return self.lib.bf_cuda_runtime_resident_bytes(self.handle)

    def infer(self, frame) -> Detections:
        """frame: a FrameInput, or a dict of host arrays (frame_scene.frame)."""
        keep = None
        if not isinstance(frame, FrameInput):
            frame, keep = frame_input(frame)
        dets, err = Detections(), _err()
        _check(self.lib.bf_cuda_runtime_infer(self.handle, C.byref(frame), C.byref(dets), err,
                                              512), err, "bf_cuda_runtime_infer")
        del keep
        return dets

    def debug_bev_stats(self):
        out, err = (C.c_float * 4)(), _err()
        _check(self.lib.bf_cuda_runtime_debug_bev_stats(self.handle, out, err, 512), err,
               "bf_cuda_runtime_debug_bev_stats")
        return list(out)

    def debug_hashes(self):
        out, err = (C.c_ulonglong * 11)(), _err()
        _check(self.lib.bf_cuda_runtime_debug_hashes(self.handle, out, err, 512), err,
               "bf_cuda_runtime_debug_hashes")
        return list(out)

    def debug_fail_next(self):
        """Arm a one-shot failure of the next infer after its calibration
        upload (bfhip_debug_runtime_fail_next, include/bfhip_debug.h)."""
        err = _err()
        _check(self.lib.bfhip_debug_runtime_fail_next(self.handle, err, 512), err,
               "bfhip_debug_runtime_fail_next")
