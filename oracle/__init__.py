"""ctypes binding of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker.  The same wrapper drives
four interchangeable libraries with identical C signatures:

  ``port``        oracle/_build/liboracle.so         restatement, OpenMP dispatch
  ``port_scalar`` oracle/_build/liboracle_scalar.so  restatement, no OpenMP
  ``ref``         oracle/_ref/libbfref.so            reference C compiled from its sources
  ``ref_scalar``  oracle/_ref/libbfref_scalar.so     same, no OpenMP
  ``ref_o3``      oracle/_ref/libbfref_o3.so         reference C under its own -O3 CFLAGS
                                                     (timed CPU baseline only)

Each library carries its own BFW reader, so models are opened through the
library that consumes them.
"""

from __future__ import annotations

import ctypes as C
import os
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIBS = {
    "port": HERE / "_build" / "liboracle.so",
    "port_scalar": HERE / "_build" / "liboracle_scalar.so",
    "ref": HERE / "_ref" / "libbfref.so",
    "ref_scalar": HERE / "_ref" / "libbfref_scalar.so",
    "ref_o3": HERE / "_ref" / "libbfref_o3.so",
}

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_sz = C.c_size_t


class ConvDesc(C.Structure):
    _fields_ = [(n, _sz) for n in (
        "n", "in_channels", "in_height", "in_width", "out_channels", "kernel_height",
        "kernel_width", "stride_height", "stride_width", "pad_height", "pad_width",
        "dilation_height", "dilation_width", "groups")]


class ConvTransposeDesc(C.Structure):
    _fields_ = [(n, _sz) for n in (
        "n", "in_channels", "in_height", "in_width", "out_channels", "kernel_height",
        "kernel_width", "stride_height", "stride_width", "pad_height", "pad_width",
        "output_pad_height", "output_pad_width", "dilation_height", "dilation_width",
        "groups")]


class WindowDesc(C.Structure):
    _fields_ = [(n, _sz) for n in (
        "batches", "height", "width", "channels", "heads", "window_size", "shift_size")]


class LssDesc(C.Structure):
    """bf_lss_desc (include/bf_lss.h)."""
    _fields_ = [("batches", _sz), ("cameras", _sz), ("depth_bins", _sz),
                ("feature_height", _sz), ("feature_width", _sz), ("channels", _sz),
                ("grid_minimum", C.c_float * 3), ("grid_step", C.c_float * 3),
                ("grid_cells", _sz * 3)]


def lss_desc(batches, cameras, depth_bins, height, width, channels, minimum, step, cells):
    return LssDesc(batches, cameras, depth_bins, height, width, channels,
                   (C.c_float * 3)(*minimum), (C.c_float * 3)(*step), (_sz * 3)(*cells))


class OracleError(RuntimeError):
    pass


class TfRaw(C.Structure):
    """bf_transfusion_raw_outputs (include/bf_transfusion_decoder.h)."""
    _fields_ = [(n, C.c_void_p) for n in (
        "center", "height", "dimension_log", "rotation", "velocity", "heatmap_logits",
        "query_scores", "labels", "indices")]


class VoxelConfig(C.Structure):
    """bf_voxel_config (include/bf_voxel.h)."""
    _fields_ = [("minimum", C.c_float * 3), ("maximum", C.c_float * 3),
                ("voxel_size", C.c_float * 3), ("point_features", C.c_size_t),
                ("max_points_per_voxel", C.c_size_t), ("max_voxels", C.c_size_t)]


class VoxelStats(C.Structure):
    """bf_voxel_stats (include/bf_voxel.h)."""
    _fields_ = [(n, C.c_size_t) for n in (
        "input_points", "accepted_points", "rejected_nonfinite", "rejected_out_of_range",
        "dropped_voxel_capacity", "dropped_point_capacity")]


class SparseDesc(C.Structure):
    """bf_sparse_conv3d_desc (reference include/bf_kernels.h:37-46)."""
    _fields_ = [(n, C.c_size_t) for n in (
        "batches", "in_depth", "in_height", "in_width", "in_channels", "out_channels",
        "kernel_depth", "kernel_height", "kernel_width", "stride_depth", "stride_height",
        "stride_width", "pad_depth", "pad_height", "pad_width", "dilation_depth",
        "dilation_height", "dilation_width")] + [("submanifold", C.c_int)]


def voxel_config(max_voxels, minimum=(-54.0, -54.0, -5.0), maximum=(54.0, 54.0, 3.0),
                 size=(0.075, 0.075, 0.2), features=5, max_points=10):
    """The runtime's voxel contract (runtime.c:262-265) by default."""
    return VoxelConfig((C.c_float * 3)(*minimum), (C.c_float * 3)(*maximum),
                       (C.c_float * 3)(*size), features, max_points, max_voxels)


class Detection(C.Structure):
    """bf_detection (include/bevfusion.h)."""
    _fields_ = [(n, C.c_float) for n in ("x", "y", "z", "width", "length", "height", "yaw",
                                         "velocity_x", "velocity_y", "score")] + \
               [("class_id", C.c_int)]


class Detections(C.Structure):
    """bf_detections (include/bevfusion.h)."""
    _fields_ = [("items", Detection * 200), ("count", C.c_int)]


class FrameInput(C.Structure):
    """bf_frame_input (reference include/bf_runtime.h:14-27)."""
    _fields_ = [("camera_images", C.c_void_p), ("points", C.c_void_p),
                ("point_count", C.c_size_t), ("camera_intrinsics_6x16", C.c_void_p),
                ("camera_to_lidar_6x16", C.c_void_p), ("image_augmentation_6x16", C.c_void_p),
                ("lidar_augmentation_16", C.c_void_p), ("lidar_to_image_6x16", C.c_void_p)]


def detections_array(d):
    """bf_detections -> float64 array [count, 11]."""
    rows = [[getattr(d.items[i], f) for f, _ in Detection._fields_] for i in range(d.count)]
    return np.array(rows, np.float64).reshape(-1, 11)


def available(flavour: str) -> bool:
    return LIBS[flavour].exists()


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class Oracle:
    def __init__(self, flavour: str = "port"):
        path = LIBS[flavour]
        if not path.exists():
            raise OracleError(f"oracle library {path} is not built")
        self.flavour = flavour
        self.lib = C.CDLL(str(path))
        L = self.lib
        L.bf_model_open.argtypes = [C.c_char_p, C.POINTER(C.c_void_p), C.c_char_p, _sz]
        L.bf_model_close.argtypes = [C.c_void_p]
        L.bf_cpu_kernel_backend.restype = C.c_char_p
        L.bf_conv2d_f32.argtypes = [_f32p, _f32p, C.c_void_p, _f32p, C.POINTER(ConvDesc)]
        L.bf_conv2d_f32_ref.argtypes = L.bf_conv2d_f32.argtypes
        L.bf_conv2d_output_shape.argtypes = [C.POINTER(ConvDesc), C.POINTER(_sz), C.POINTER(_sz)]
        L.bf_conv_transpose2d_f32_ref.argtypes = [_f32p, _f32p, C.c_void_p, _f32p,
                                                  C.POINTER(ConvTransposeDesc)]
        L.bf_conv_transpose2d_output_shape.argtypes = [C.POINTER(ConvTransposeDesc),
                                                       C.POINTER(_sz), C.POINTER(_sz)]
        for n in ("bf_linear_f32", "bf_linear_f32_ref"):
            getattr(L, n).argtypes = [_f32p, _f32p, C.c_void_p, _f32p, _sz, _sz, _sz]
            getattr(L, n).restype = None
        for n in ("bf_layer_norm_f32", "bf_layer_norm_f32_ref"):
            getattr(L, n).argtypes = [_f32p, _f32p, _f32p, C.c_float, _f32p, _sz, _sz]
            getattr(L, n).restype = None
        for n in ("bf_batch_norm_2d_f32", "bf_batch_norm_2d_f32_ref"):
            getattr(L, n).argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, C.c_float, _f32p,
                                      _sz, _sz, _sz, _sz]
            getattr(L, n).restype = None
        L.bf_softmax_f32_ref.argtypes = [_f32p, _f32p, _sz, _sz]
        L.bf_softmax_f32_ref.restype = None
        for n in ("bf_gelu_f32", "bf_gelu_f32_ref", "bf_relu_f32", "bf_relu_f32_ref"):
            getattr(L, n).argtypes = [_f32p, _f32p, _sz]
            getattr(L, n).restype = None
        L.bf_swin_shifted_window_f32_ref.argtypes = [
            _f32p, _f32p, _f32p, _f32p, _i64p, _f32p, _f32p, _f32p, C.POINTER(WindowDesc)]
        L.bf_swin_shifted_window_workspace_bytes.argtypes = [C.POINTER(WindowDesc)]
        L.bf_swin_shifted_window_workspace_bytes.restype = _sz
        L.bf_swin_shifted_window_f32_workspace_ref.argtypes = [
            _f32p, _f32p, _f32p, _f32p, _i64p, _f32p, _f32p, _f32p, C.POINTER(WindowDesc),
            C.c_void_p, _sz]
        L.bf_swin_window_attention_f32_ref.argtypes = [
            _f32p, _f32p, _f32p, _f32p, _i64p, C.c_void_p, _sz, _f32p, _f32p, _f32p,
            _sz, _sz, _sz, _sz, _sz]
        for mod in ("swin_backbone", "image_fpn", "depth_head", "lss_downsample", "bev_stage",
                    "transfusion_decoder"):
            getattr(L, f"bf_{mod}_create").argtypes = [C.c_void_p, C.POINTER(C.c_void_p),
                                                       C.c_char_p, _sz]
            getattr(L, f"bf_{mod}_destroy").argtypes = [C.c_void_p]
            getattr(L, f"bf_{mod}_destroy").restype = None
        L.bf_swin_backbone_workspace_bytes.argtypes = [_sz, _sz, _sz]
        L.bf_swin_backbone_workspace_bytes.restype = _sz
        L.bf_swin_backbone_forward_ref.argtypes = [
            C.c_void_p, _f32p, _sz, _sz, _sz, _f32p, _f32p, _f32p, C.c_void_p, _sz,
            C.c_char_p, _sz]
        for mod in ("image_fpn", "depth_head", "lss_downsample"):
            getattr(L, f"bf_{mod}_workspace_bytes").argtypes = [_sz, _sz]
            getattr(L, f"bf_{mod}_workspace_bytes").restype = _sz
        L.bf_image_fpn_forward_ref.argtypes = [
            C.c_void_p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _f32p, _f32p, C.c_void_p, _sz,
            C.c_char_p, _sz]
        L.bf_depth_head_forward_ref.argtypes = [
            C.c_void_p, _f32p, _f32p, _sz, _sz, _sz, _f32p, _f32p, C.c_void_p, _sz,
            C.c_char_p, _sz]
        L.bf_lss_downsample_forward_ref.argtypes = [
            C.c_void_p, _f32p, _sz, _sz, _sz, _f32p, C.c_void_p, _sz, C.c_char_p, _sz]
        L.bf_bev_stage_workspace_bytes.argtypes = [_sz, _sz]
        L.bf_bev_stage_workspace_bytes.restype = _sz
        L.bf_bev_stage_forward_ref.argtypes = [
            C.c_void_p, _f32p, _sz, _sz, _sz, _f32p, _f32p, _f32p, C.c_void_p, _sz,
            C.c_char_p, _sz]
        L.bf_transfusion_decoder_workspace_bytes.argtypes = [_sz, _sz, _sz]
        L.bf_transfusion_decoder_workspace_bytes.restype = _sz
        L.bf_transfusion_decoder_forward_ref.argtypes = [
            C.c_void_p, _f32p, _f32p, _sz, _sz, _sz, _sz, C.c_void_p, C.c_void_p, _sz,
            C.c_char_p, _sz]
        L.bf_transfusion_select_proposals_f32_ref.argtypes = [
            _f32p, _f32p, _f32p, C.c_void_p, C.c_void_p, _sz, _sz, _sz, _sz, _sz, _sz]
        L.bf_transfusion_decode_raw_f32_ref.argtypes = [
            _f32p, _f32p, C.c_void_p, _f32p, _f32p, _f32p, _f32p, C.c_void_p, _f32p, _f32p,
            C.c_void_p, _sz, _sz, _sz, C.c_float, _f32p, _f32p]
        L.bf_transfusion_filter_detections.argtypes = [
            _f32p, _f32p, C.c_void_p, _sz, _sz, C.c_float, _f32p, C.c_void_p]
        L.bf_lss_geometry_f32_ref.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                              C.c_void_p, C.c_void_p, _f32p, _sz, _sz, _sz,
                                              _sz, _sz]
        L.bf_lss_lift_f32_ref.argtypes = [_f32p, _f32p, _f32p, C.POINTER(LssDesc)]
        L.bf_lss_bev_pool_f32_ref.argtypes = [_f32p, _f32p, _f32p, C.POINTER(LssDesc)]
        L.bf_lss_lift_pool_f32_ref.argtypes = [_f32p, _f32p, _f32p, _f32p, C.POINTER(LssDesc)]
        if hasattr(L, "bf_oracle_lss_ranks"):
            L.bf_oracle_lss_ranks.argtypes = [_f32p, C.c_void_p, C.POINTER(LssDesc)]
        # LiDAR side (depth raster, voxeliser, MeanVFE, sparse conv, backbone).
        L.bf_depth_rasterize_f32_ref.argtypes = [_f32p, _sz, _sz, _f32p, _f32p, _f32p, _f32p,
                                                 _sz, _sz, _sz, _sz]
        L.bf_voxelize_workspace_bytes.argtypes = [C.POINTER(VoxelConfig)]
        L.bf_voxelize_workspace_bytes.restype = _sz
        L.bf_voxelize_f32_workspace_ref.argtypes = [
            _f32p, _sz, _sz, C.c_int32, C.POINTER(VoxelConfig), _f32p, C.c_void_p, C.c_void_p,
            C.POINTER(_sz), C.POINTER(VoxelStats), C.c_void_p, _sz]
        L.bf_mean_vfe_f32_ref.argtypes = [_f32p, C.c_void_p, _f32p, _sz, _sz, _sz]
        L.bf_mean_vfe_f32_ref.restype = None
        L.bf_sparse_conv3d_workspace_bytes.argtypes = [_sz, _sz]
        L.bf_sparse_conv3d_workspace_bytes.restype = _sz
        L.bf_sparse_conv3d_output_shape.argtypes = [C.POINTER(SparseDesc), C.POINTER(_sz),
                                                    C.POINTER(_sz), C.POINTER(_sz)]
        L.bf_sparse_conv3d_f32_workspace_ref.argtypes = [
            C.c_void_p, _f32p, _sz, _f32p, C.c_void_p, C.c_void_p, _f32p, _sz, C.POINTER(_sz),
            C.POINTER(SparseDesc), C.c_void_p, _sz]
        L.bf_lidar_backbone_create.argtypes = [C.c_void_p, C.POINTER(C.c_void_p), C.c_char_p, _sz]
        L.bf_lidar_backbone_destroy.argtypes = [C.c_void_p]
        L.bf_lidar_backbone_destroy.restype = None
        L.bf_lidar_backbone_workspace_bytes.argtypes = [_sz]
        L.bf_lidar_backbone_workspace_bytes.restype = _sz
        L.bf_lidar_backbone_output_shape.argtypes = [_sz, _sz, _sz, C.POINTER(_sz),
                                                     C.POINTER(_sz), C.POINTER(_sz)]
        L.bf_lidar_backbone_forward_ref.argtypes = [
            C.c_void_p, C.c_void_p, _f32p, _sz, _sz, _sz, _sz, _sz, _sz, _f32p, C.c_void_p, _sz,
            C.c_char_p, _sz]

    # ---- utilities -------------------------------------------------------
    def backend(self) -> str:
        return self.lib.bf_cpu_kernel_backend().decode()

    def open_model(self, path):
        handle, err = C.c_void_p(), C.create_string_buffer(256)
        if not self.lib.bf_model_open(str(path).encode(), C.byref(handle), err, 256):
            raise OracleError(err.value.decode())
        return _Model(self.lib, handle)

    # ---- operators -------------------------------------------------------
    def conv2d(self, x, w, b, stride=(1, 1), pad=(0, 0), dilation=(1, 1), groups=1,
               scalar=False):
        x, w = _f32(x), _f32(w)
        n, ci, ih, iw = x.shape
        co, _, kh, kw = w.shape
        d = ConvDesc(n, ci, ih, iw, co, kh, kw, stride[0], stride[1], pad[0], pad[1],
                     dilation[0], dilation[1], groups)
        oh, ow = _sz(), _sz()
        if not self.lib.bf_conv2d_output_shape(C.byref(d), C.byref(oh), C.byref(ow)):
            raise OracleError("invalid convolution")
        y = np.empty((n, co, oh.value, ow.value), np.float32)
        bb = None if b is None else _f32(b)
        fn = self.lib.bf_conv2d_f32_ref if scalar else self.lib.bf_conv2d_f32
        if not fn(x, w, None if bb is None else bb.ctypes.data, y, C.byref(d)):
            raise OracleError("convolution failed")
        return y

    def conv_transpose2d(self, x, w_iohw, b, stride=(1, 1), pad=(0, 0), output_pad=(0, 0),
                         dilation=(1, 1), groups=1):
        x, w = _f32(x), _f32(w_iohw)
        n, ci, ih, iw = x.shape
        co = w.shape[1] * groups
        d = ConvTransposeDesc(n, ci, ih, iw, co, w.shape[2], w.shape[3], stride[0], stride[1],
                              pad[0], pad[1], output_pad[0], output_pad[1], dilation[0],
                              dilation[1], groups)
        oh, ow = _sz(), _sz()
        if not self.lib.bf_conv_transpose2d_output_shape(C.byref(d), C.byref(oh), C.byref(ow)):
            raise OracleError("invalid transposed convolution")
        y = np.empty((n, co, oh.value, ow.value), np.float32)
        bb = None if b is None else _f32(b)
        if not self.lib.bf_conv_transpose2d_f32_ref(x, w, None if bb is None else bb.ctypes.data,
                                                    y, C.byref(d)):
            raise OracleError("transposed convolution failed")
        return y

    def linear(self, x, w, b, scalar=False):
        x, w = _f32(x), _f32(w)
        rows, k = x.shape
        y = np.empty((rows, w.shape[0]), np.float32)
        bb = None if b is None else _f32(b)
        fn = self.lib.bf_linear_f32_ref if scalar else self.lib.bf_linear_f32
        fn(x, w, None if bb is None else bb.ctypes.data, y, rows, k, w.shape[0])
        return y

    def layer_norm(self, x, g, b, eps=1e-5, scalar=False):
        x = _f32(x)
        y = np.empty_like(x)
        fn = self.lib.bf_layer_norm_f32_ref if scalar else self.lib.bf_layer_norm_f32
        fn(x, _f32(g), _f32(b), eps, y, x.size // x.shape[-1], x.shape[-1])
        return y

    def batch_norm(self, x, g, b, mean, var, eps=1e-5, scalar=False):
        x = _f32(x)
        y = np.empty_like(x)
        fn = self.lib.bf_batch_norm_2d_f32_ref if scalar else self.lib.bf_batch_norm_2d_f32
        fn(x, _f32(g), _f32(b), _f32(mean), _f32(var), eps, y, *x.shape)
        return y

    def softmax(self, x):
        x = _f32(x)
        y = np.empty_like(x)
        self.lib.bf_softmax_f32_ref(x, y, x.size // x.shape[-1], x.shape[-1])
        return y

    def gelu(self, x, scalar=False):
        x = _f32(x)
        y = np.empty_like(x)
        (self.lib.bf_gelu_f32_ref if scalar else self.lib.bf_gelu_f32)(x, y, x.size)
        return y

    def relu(self, x):
        x = _f32(x)
        y = np.empty_like(x)
        self.lib.bf_relu_f32(x, y, x.size)
        return y

    def swin_window(self, query, qkv_w, qkv_b, rel_bias, rel_index, proj_w, proj_b,
                    heads, window, shift, streamed=True):
        """One W-MSA / SW-MSA branch on [B,H,W,C] tokens (swin.c:119-311)."""
        q = _f32(query)
        b, h, w, c = q.shape
        d = WindowDesc(b, h, w, c, heads, window, shift)
        out = np.zeros_like(q)
        args = (q, _f32(qkv_w), _f32(qkv_b), _f32(rel_bias),
                np.ascontiguousarray(rel_index, np.int64), _f32(proj_w), _f32(proj_b), out,
                C.byref(d))
        if streamed:
            nbytes = self.lib.bf_swin_shifted_window_workspace_bytes(C.byref(d))
            ws = np.empty(nbytes // 4 + 1, np.float32)
            ok = self.lib.bf_swin_shifted_window_f32_workspace_ref(*args, ws.ctypes.data, nbytes)
        else:
            ok = self.lib.bf_swin_shifted_window_f32_ref(*args)
        if not ok:
            raise OracleError("window attention failed")
        return out

    # ---- modules -----------------------------------------------------------
    def swin_backbone(self, model, images):
        x = _f32(images)
        b, _, ih, iw = x.shape
        net = model.create("swin_backbone")
        try:
            outs = [np.empty((b, c, -(-ih // d), -(-iw // d)), np.float32)
                    for c, d in ((192, 8), (384, 16), (768, 32))]
            nbytes = self.lib.bf_swin_backbone_workspace_bytes(b, ih, iw)
            ws = np.empty(nbytes // 4 + 1, np.float32)
            err = C.create_string_buffer(256)
            if not self.lib.bf_swin_backbone_forward_ref(net, x, b, ih, iw, *outs, ws.ctypes.data,
                                                         nbytes, err, 256):
                raise OracleError(err.value.decode())
            return tuple(outs)
        finally:
            self.lib.bf_swin_backbone_destroy(net)

    def image_fpn(self, model, s0, s1, s2):
        s0, s1, s2 = _f32(s0), _f32(s1), _f32(s2)
        b, _, h, w = s0.shape
        net = model.create("image_fpn")
        try:
            o0 = np.empty((b, 256, h, w), np.float32)
            o1 = np.empty((b, 256, (h + 1) // 2, (w + 1) // 2), np.float32)
            nbytes = self.lib.bf_image_fpn_workspace_bytes(h, w)
            ws = np.empty(nbytes // 4 + 1, np.float32)
            err = C.create_string_buffer(256)
            if not self.lib.bf_image_fpn_forward_ref(net, s0, s1, s2, b, h, w, o0, o1,
                                                     ws.ctypes.data, nbytes, err, 256):
                raise OracleError(err.value.decode())
            return o0, o1
        finally:
            self.lib.bf_image_fpn_destroy(net)

    def depth_head(self, model, features, depth):
        f, d = _f32(features), _f32(depth)
        b, _, h, w = f.shape
        net = model.create("depth_head")
        try:
            logits = np.empty((b, 118, h, w), np.float32)
            ctx = np.empty((b, 80, h, w), np.float32)
            nbytes = self.lib.bf_depth_head_workspace_bytes(h, w)
            ws = np.empty(nbytes // 4 + 1, np.float32)
            err = C.create_string_buffer(256)
            if not self.lib.bf_depth_head_forward_ref(net, f, d, b, h, w, logits, ctx,
                                                      ws.ctypes.data, nbytes, err, 256):
                raise OracleError(err.value.decode())
            return logits, ctx
        finally:
            self.lib.bf_depth_head_destroy(net)

    def lss_downsample(self, model, bev):
        x = _f32(bev)
        b, _, h, w = x.shape
        net = model.create("lss_downsample")
        try:
            out = np.empty((b, 80, w // 2, h // 2), np.float32)
            nbytes = self.lib.bf_lss_downsample_workspace_bytes(h, w)
            ws = np.empty(nbytes // 4 + 1, np.float32)
            err = C.create_string_buffer(256)
            if not self.lib.bf_lss_downsample_forward_ref(net, x, b, h, w, out, ws.ctypes.data,
                                                          nbytes, err, 256):
                raise OracleError(err.value.decode())
            return out
        finally:
            self.lib.bf_lss_downsample_destroy(net)


    # ---- BEV stage (bf_bev_stage.h) --------------------------------------
    def bev_stage(self, model, x):
        """x [B,336,H,W] -> (spatial [B,512,H,W], shared [B,128,H,W],
        heatmap [B,10,H,W])."""
        x = _f32(x)
        b, c, h, w = x.shape
        net = model.create("bev_stage")
        try:
            nbytes = self.lib.bf_bev_stage_workspace_bytes(h, w)
            ws = np.empty(max(nbytes, 1), np.uint8)
            sp = np.empty((b, 512, h, w), np.float32)
            sh = np.empty((b, 128, h, w), np.float32)
            hm = np.empty((b, 10, h, w), np.float32)
            err = C.create_string_buffer(256)
            if not self.lib.bf_bev_stage_forward_ref(net, x, b, h, w, sp, sh, hm, ws.ctypes.data,
                                                     nbytes, err, 256):
                raise OracleError(err.value.decode())
        finally:
            self.lib.bf_bev_stage_destroy(net)
        return sp, sh, hm

    # ---- LiDAR side --------------------------------------------------------
    def depth_raster(self, points_b, lidar_aug, lidar_to_image, image_aug, cameras, height,
                     width, batches=1):
        """points [P, stride] with column 0 = batch -> dense depth [B,N,H,W]
        (depth_raster.c:49-105)."""
        pts = _f32(points_b)
        out = np.empty((batches, cameras, height, width), np.float32)
        if not self.lib.bf_depth_rasterize_f32_ref(
                pts if pts.size else np.zeros((1, pts.shape[1]), np.float32), pts.shape[0],
                pts.shape[1], _f32(lidar_aug), _f32(lidar_to_image), _f32(image_aug), out,
                batches, cameras, height, width):
            raise OracleError("depth raster failed")
        return out

    def voxelize(self, points, config, batch=0):
        """points [P, F] -> (voxels [V,M,F], coords int32 [V,4], counts int64 [V], stats)."""
        pts = _f32(points)
        M, F, cap = config.max_points_per_voxel, config.point_features, config.max_voxels
        voxels = np.empty((cap, M, F), np.float32)
        coords = np.empty((cap, 4), np.int32)
        counts = np.empty((cap,), np.int64)
        n, st = _sz(0), VoxelStats()
        nbytes = self.lib.bf_voxelize_workspace_bytes(C.byref(config))
        ws = np.empty(max(nbytes, 1), np.uint8)
        if not self.lib.bf_voxelize_f32_workspace_ref(
                pts if pts.size else np.zeros((1, F), np.float32), pts.shape[0], pts.shape[1],
                batch, C.byref(config), voxels, coords.ctypes.data, counts.ctypes.data,
                C.byref(n), C.byref(st), ws.ctypes.data, nbytes):
            raise OracleError("voxelize failed")
        v = n.value
        return voxels[:v], coords[:v], counts[:v], st

    def mean_vfe(self, voxels, counts):
        v, m, c = voxels.shape
        out = np.empty((v, c), np.float32)
        cnt = np.ascontiguousarray(counts, np.int64)
        self.lib.bf_mean_vfe_f32_ref(_f32(voxels), cnt.ctypes.data, out, v, m, c)
        return out

    def sparse_conv3d(self, coords, features, weight, bias, desc, capacity):
        """coords int32 [N,4], features [N,Ci], weight [kd,kh,kw,Ci,Co] ->
        (coords [M,4], features [M,Co])."""
        coords = np.ascontiguousarray(coords, np.int32)
        feats = _f32(features)
        oc = np.empty((capacity, 4), np.int32)
        of = np.empty((capacity, desc.out_channels), np.float32)
        n = _sz(0)
        nbytes = self.lib.bf_sparse_conv3d_workspace_bytes(coords.shape[0], capacity)
        ws = np.empty(max(nbytes, 1), np.uint8)
        b = None if bias is None else _f32(bias)
        if not self.lib.bf_sparse_conv3d_f32_workspace_ref(
                coords.ctypes.data, feats, coords.shape[0], _f32(weight),
                None if b is None else b.ctypes.data, oc.ctypes.data, of, capacity, C.byref(n),
                C.byref(desc), ws.ctypes.data, nbytes):
            raise OracleError("sparse conv3d failed")
        return oc[:n.value], of[:n.value]

    def lidar_backbone(self, model, coords, features, depth=41, height=1440, width=1440,
                       capacity=None, batches=1):
        """voxel coords int32 [N,4] + MeanVFE features [N,5] -> dense
        [B,128,D',H',W'] (lidar_backbone.c:191-273)."""
        coords = np.ascontiguousarray(coords, np.int32)
        feats = _f32(features)
        cap = capacity or 8 * coords.shape[0]
        od, oh, ow = _sz(), _sz(), _sz()
        if not self.lib.bf_lidar_backbone_output_shape(depth, height, width, C.byref(od),
                                                       C.byref(oh), C.byref(ow)):
            raise OracleError("lidar backbone output shape")
        dense = np.empty((batches, 128, od.value, oh.value, ow.value), np.float32)
        nbytes = self.lib.bf_lidar_backbone_workspace_bytes(cap)
        ws = np.empty(max(nbytes, 1), np.uint8)
        err = C.create_string_buffer(256)
        net = model.create("lidar_backbone")
        try:
            if not self.lib.bf_lidar_backbone_forward_ref(
                    net, coords.ctypes.data, feats, coords.shape[0], batches, depth, height, width,
                    cap, dense, ws.ctypes.data, nbytes, err, 256):
                raise OracleError(err.value.decode())
        finally:
            self.lib.bf_lidar_backbone_destroy(net)
        return dense

    # ---- TransFusion head ------------------------------------------------
    TF_FIELDS = (("center", 2), ("height", 1), ("dimension_log", 3), ("rotation", 2),
                 ("velocity", 2), ("heatmap_logits", 10), ("query_scores", 10))

    def transfusion(self, model, shared, heatmap, proposals):
        """shared [B,128,H,W], heatmap logits [B,10,H,W] -> dict of raw outputs
        (channel-major [B,C,P] arrays, int64 labels / indices [B,P])."""
        shared, heatmap = _f32(shared), _f32(heatmap)
        b, _, h, w = shared.shape
        outs = {k: np.empty((b, c, proposals), np.float32) for k, c in self.TF_FIELDS}
        outs["labels"] = np.empty((b, proposals), np.int64)
        outs["indices"] = np.empty((b, proposals), np.int64)
        raw = TfRaw(*[outs[k].ctypes.data for k, _ in self.TF_FIELDS],
                    outs["labels"].ctypes.data, outs["indices"].ctypes.data)
        net = model.create("transfusion_decoder")
        try:
            nbytes = self.lib.bf_transfusion_decoder_workspace_bytes(h, w, proposals)
            ws = np.empty(max(nbytes, 1), np.uint8)
            err = C.create_string_buffer(256)
            if not self.lib.bf_transfusion_decoder_forward_ref(
                    net, shared, heatmap, b, h, w, proposals, C.byref(raw), ws.ctypes.data,
                    nbytes, err, 256):
                raise OracleError(err.value.decode())
        finally:
            self.lib.bf_transfusion_decoder_destroy(net)
        return outs

    def transfusion_detections(self, outs, threshold, stride=8.0, voxel=(0.075, 0.075),
                               minimum=(-54.0, -54.0),
                               post_range=(-61.2, -61.2, -10.0, 61.2, 61.2, 10.0)):
        """decode_raw + filter (transfusion.c:134-193) -> list of per-batch
        detection arrays [n, 11] (x y z w l h yaw vx vy score class)."""
        b, _, p = outs["center"].shape
        boxes = np.empty((b, p, 9), np.float32)
        scores = np.empty((b, p), np.float32)
        labels = np.empty((b, p), np.int64)
        if not self.lib.bf_transfusion_decode_raw_f32_ref(
                outs["heatmap_logits"], outs["query_scores"], outs["labels"].ctypes.data,
                outs["center"], outs["height"], outs["dimension_log"], outs["rotation"],
                outs["velocity"].ctypes.data, boxes, scores, labels.ctypes.data, b, 10, p,
                stride, _f32(voxel), _f32(minimum)):
            raise OracleError("TransFusion decode failed")
        dets = (Detections * b)()
        if not self.lib.bf_transfusion_filter_detections(boxes, scores, labels.ctypes.data, b, p,
                                                         threshold, _f32(post_range), dets):
            raise OracleError("TransFusion filter failed")
        return [detections_array(d) for d in dets]

    # ---- frame runtime (bf_runtime.h) --------------------------------------
    def runtime_infer(self, model_path, frame, point_capacity=300000, voxel_capacity=160000,
                      sparse_capacity=160000):
        """The CPU frame runtime (runtime.c:238-413) on a dict of host arrays
        (images, points, camera_intrinsics, camera_to_lidar, image_augmentation,
        lidar_augmentation, lidar_to_image) -> bf_detections."""
        L = self.lib
        L.bf_runtime_create.argtypes = [C.c_char_p, C.POINTER(C.c_void_p), C.c_char_p, _sz]
        L.bf_runtime_destroy.argtypes = [C.c_void_p]
        L.bf_runtime_destroy.restype = None
        L.bf_runtime_workspace_bytes.argtypes = [_sz, _sz, _sz]
        L.bf_runtime_workspace_bytes.restype = _sz
        L.bf_runtime_infer_cpu_ref.argtypes = [C.c_void_p, C.POINTER(FrameInput), _sz, _sz, _sz,
                                               C.POINTER(Detections), C.c_void_p, _sz,
                                               C.c_char_p, _sz]
        keys = ("images", "points", "camera_intrinsics", "camera_to_lidar", "image_augmentation",
                "lidar_augmentation", "lidar_to_image")
        arrs = {k: _f32(frame[k]) for k in keys}
        fi = FrameInput(*[arrs[k].ctypes.data for k in keys[:2]], arrs["points"].shape[0],
                        *[arrs[k].ctypes.data for k in keys[2:]])
        handle, err = C.c_void_p(), C.create_string_buffer(256)
        if not L.bf_runtime_create(str(model_path).encode(), C.byref(handle), err, 256):
            raise OracleError(err.value.decode())
        try:
            nbytes = L.bf_runtime_workspace_bytes(point_capacity, voxel_capacity, sparse_capacity)
            if not nbytes:
                raise OracleError("invalid runtime capacities")
            ws = np.empty(nbytes, np.uint8)
            dets = Detections()
            if not L.bf_runtime_infer_cpu_ref(handle, C.byref(fi), point_capacity, voxel_capacity,
                                              sparse_capacity, C.byref(dets), ws.ctypes.data,
                                              nbytes, err, 256):
                raise OracleError(err.value.decode())
        finally:
            L.bf_runtime_destroy(handle)
        return dets

    # ---- lift-splat pooling (bf_lss.h) ------------------------------------
    def lss_geometry(self, frustum, cam_rot, cam_trans, intrinsics, post_rot, post_trans,
                     extra_rot=None, extra_trans=None):
        """frustum [D,H,W,3]; per-camera matrices [B,N,3,3] / [B,N,3]; optional
        per-batch extra [B,3,3] / [B,3].  Returns geometry [B,N,D,H,W,3]."""
        fr = _f32(frustum)
        b, n = cam_rot.shape[:2]
        d, h, w = fr.shape[:3]
        out = np.empty((b, n, d, h, w, 3), np.float32)
        er = None if extra_rot is None else _f32(extra_rot)
        et = None if extra_trans is None else _f32(extra_trans)
        if not self.lib.bf_lss_geometry_f32_ref(
                fr, _f32(cam_rot), _f32(cam_trans), _f32(intrinsics), _f32(post_rot),
                _f32(post_trans), None if er is None else er.ctypes.data,
                None if et is None else et.ctypes.data, out, b, n, d, h, w):
            raise OracleError("LSS geometry failed (singular matrix)")
        return out

    def lss_lift(self, logits, context, desc):
        out = np.empty(tuple(logits.shape) + (desc.channels,), np.float32)
        if not self.lib.bf_lss_lift_f32_ref(_f32(logits), _f32(context), out, C.byref(desc)):
            raise OracleError("LSS lift failed")
        return out

    @staticmethod
    def _bev_shape(desc):
        return (desc.batches, desc.channels * desc.grid_cells[2], desc.grid_cells[0],
                desc.grid_cells[1])

    def lss_bev_pool(self, lifted, geometry, desc):
        out = np.empty(self._bev_shape(desc), np.float32)
        if not self.lib.bf_lss_bev_pool_f32_ref(_f32(lifted), _f32(geometry), out, C.byref(desc)):
            raise OracleError("LSS pool failed")
        return out

    def lss_ranks(self, geometry, desc):
        """Per-sample cell rank within its batch, -1 outside (int32)."""
        g = _f32(geometry)
        out = np.empty(g.shape[:-1], np.int32)
        if not self.lib.bf_oracle_lss_ranks(g, out.ctypes.data, C.byref(desc)):
            raise OracleError("LSS ranks failed")
        return out

    def lss_lift_pool(self, logits, context, geometry, desc):
        out = np.empty(self._bev_shape(desc), np.float32)
        if not self.lib.bf_lss_lift_pool_f32_ref(_f32(logits), _f32(context), _f32(geometry),
                                                 out, C.byref(desc)):
            raise OracleError("LSS lift-pool failed")
        return out


class _Model:
    def __init__(self, lib, handle):
        self.lib, self.handle = lib, handle

    def create(self, module: str):
        out, err = C.c_void_p(), C.create_string_buffer(256)
        if not getattr(self.lib, f"bf_{module}_create")(self.handle, C.byref(out), err, 256):
            raise OracleError(err.value.decode())
        return out

    def close(self):
        if self.handle:
            self.lib.bf_model_close(self.handle)
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


def scalar_env():
    """Context manager forcing BF_CPU_SCALAR=1 (the reference's scalar switch)."""
    class _Env:
        def __enter__(self):
            self.prev = os.environ.get("BF_CPU_SCALAR")
            os.environ["BF_CPU_SCALAR"] = "1"

        def __exit__(self, *exc):
            if self.prev is None:
                os.environ.pop("BF_CPU_SCALAR", None)
            else:
                os.environ["BF_CPU_SCALAR"] = self.prev
    return _Env()
