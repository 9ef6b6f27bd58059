"""BFW container writer and synthetic camera-branch checkpoints.

The writer emits the layout read by ``csrc/bfw_model.c`` (and by the
reference's ``src/model.c``): a 64-byte header, 160-byte directory entries and
64-byte aligned little-endian payloads, as produced by the reference exporter
``tools/export_checkpoint.py:12-17,49-80``.

``camera_branch_tensors`` builds random-init weights under the exact tensor
names and shapes that the Swin-T context (reference src/cuda_swin.cu:290-317)
and the camera-neck context (src/cuda_camera.cu:301-318) bind.  There is no
network access for the real checkpoint, so every benchmark and parity test
runs on these synthetic weights.
"""

from __future__ import annotations

import pathlib
import struct
import zlib

import numpy as np

MAGIC = b"BFW0001\0"
HEADER = struct.Struct("<8sIIQQQQII8s")
ENTRY = struct.Struct("<96sII8IQQII")
ALIGN = 64
F32, I64 = 1, 2

SWIN_CHANNELS = (96, 192, 384, 768)
SWIN_HEADS = (3, 6, 12, 24)
SWIN_DEPTHS = (2, 2, 6, 2)


# --------------------------------------------------------------------------
# Counter-based RNG: splitmix64 over (stream, index) + Box-Muller.  Every
# value depends only on (seed, name, index), so a tensor regenerates
# bit-identically regardless of the order tensors are produced in.
# --------------------------------------------------------------------------
_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix64(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def stream_key(seed: int, name: str) -> int:
    return ((seed & 0xFFFFFFFF) << 32) ^ zlib.crc32(name.encode("utf-8"))


def uniform(key: int, count: int, offset: int = 0) -> np.ndarray:
    """Uniform float64 in (0, 1), 53-bit, from counter ``offset + i``."""
    idx = np.arange(offset, offset + count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        base = _splitmix64(np.uint64(key) * np.uint64(0xD1B54A32D192ED03) + idx)
    bits = _splitmix64(base) >> np.uint64(11)
    return (bits.astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)


def normal(key: int, count: int) -> np.ndarray:
    """Standard normal float64 via Box-Muller on paired uniforms."""
    pairs = (count + 1) // 2
    u1 = uniform(key, pairs, 0)
    u2 = uniform(key, pairs, 1 << 40)
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.concatenate([r * np.cos(2.0 * np.pi * u2), r * np.sin(2.0 * np.pi * u2)])
    return z[:count]


def randn(seed: int, name: str, shape, std=1.0, mean=0.0) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    return (normal(stream_key(seed, name), n) * std + mean).astype(np.float32).reshape(shape)


def randu(seed: int, name: str, shape, low=0.0, high=1.0) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    u = uniform(stream_key(seed, name), n)
    return (low + (high - low) * u).astype(np.float32).reshape(shape)


# --------------------------------------------------------------------------
# Writer
# --------------------------------------------------------------------------
def _align(v: int) -> int:
    return (v + ALIGN - 1) & -ALIGN


def write_bfw(tensors, path) -> int:
    """Write [(name, ndarray)] (float32 or int64) to ``path``; returns bytes."""
    path = pathlib.Path(path)
    entries, payloads = [], []
    data_offset = _align(HEADER.size + len(tensors) * ENTRY.size)
    cursor = data_offset
    seen = set()
    for name, arr in tensors:
        if name in seen:
            raise ValueError(f"duplicate tensor {name}")
        seen.add(name)
        arr = np.ascontiguousarray(arr)
        if arr.dtype == np.float32:
            dtype = F32
        elif arr.dtype == np.int64:
            dtype = I64
        else:
            raise TypeError(f"{name}: unsupported dtype {arr.dtype}")
        enc = name.encode("utf-8")
        if len(enc) >= 96 or arr.ndim > 8 or any(d <= 0 for d in arr.shape):
            raise ValueError(f"{name}: unsupported name or shape {arr.shape}")
        raw = arr.astype(arr.dtype.newbyteorder("<"), copy=False).tobytes()
        cursor = _align(cursor)
        dims = list(arr.shape) + [0] * (8 - arr.ndim)
        entries.append(ENTRY.pack(enc, dtype, arr.ndim, *dims, cursor, len(raw),
                                  zlib.crc32(raw) & 0xFFFFFFFF, 0))
        payloads.append((cursor, raw))
        cursor += len(raw)
    directory = b"".join(entries)
    header = HEADER.pack(MAGIC, 1, HEADER.size, len(tensors), HEADER.size,
                         data_offset, cursor, zlib.crc32(directory) & 0xFFFFFFFF,
                         0, b"\0" * 8)
    path.parent.mkdir(parents=True, exist_ok=True)
    tmp = path.with_name(path.name + ".tmp")
    with tmp.open("wb") as f:
        f.write(header)
        f.write(directory)
        for off, raw in payloads:
            f.write(b"\0" * (off - f.tell()))
            f.write(raw)
    tmp.replace(path)
    return cursor


# --------------------------------------------------------------------------
# Synthetic camera-branch checkpoint
# --------------------------------------------------------------------------
def relative_position_index(window: int = 7) -> np.ndarray:
    """Swin relative index, closed form (qy-ky+w-1)*(2w-1) + (qx-kx+w-1)."""
    t = np.arange(window * window)
    qy, qx = (t // window)[:, None], (t % window)[:, None]
    ky, kx = (t // window)[None, :], (t % window)[None, :]
    return ((qy - ky + window - 1) * (2 * window - 1) + (qx - kx + window - 1)).astype(np.int64)


class _Init:
    """Weight initialisation policy.

    ``mode="baseline"``: every weight ~N(0, 0.02), as BASELINE.json configs
    2-4 state.  ``mode="fan_in"``: weights ~N(0, gain/sqrt(fan_in)) so every
    residual branch contributes O(1) to its output; the parity tests use it
    so that a wrong branch cannot hide under the residual stream.
    """

    def __init__(self, seed: int, mode: str = "baseline", gain: float = 1.0, offset: float = 0.0):
        if mode not in ("baseline", "fan_in"):
            raise ValueError(mode)
        self.seed, self.mode, self.gain, self.offset = seed, mode, gain, offset

    def weight(self, name, shape, fan_in):
        std = 0.02 if self.mode == "baseline" else self.gain / np.sqrt(fan_in)
        return randn(self.seed, name, shape, std)

    def bias(self, name, shape):
        b = randn(self.seed, name, shape, 0.02)
        # ``offset``: the residual branches' output biases (attention proj and
        # fc2) add a common offset to every channel, so the residual rows the
        # LayerNorms see carry a mean far larger than their spread.
        if self.offset and name.endswith(("attn.w_msa.proj.bias", "ffn.layers.1.bias")):
            b = (b + self.offset).astype(np.float32)
        return b

    def norm(self, prefix, c):
        return [(prefix + ".weight", randn(self.seed, prefix + ".weight", (c,), 0.02, 1.0)),
                (prefix + ".bias", randn(self.seed, prefix + ".bias", (c,), 0.02))]

    def bn(self, prefix, c):
        return [(prefix + ".weight", randn(self.seed, prefix + ".weight", (c,), 0.1, 1.0)),
                (prefix + ".bias", randn(self.seed, prefix + ".bias", (c,), 0.1)),
                (prefix + ".running_mean", randn(self.seed, prefix + ".running_mean", (c,), 0.1)),
                (prefix + ".running_var", randu(self.seed, prefix + ".running_var", (c,), 0.5, 1.5))]


def swin_tensors(init: _Init):
    out = []
    p = "image_backbone."
    out.append((p + "patch_embed.projection.weight",
                init.weight(p + "patch_embed.projection.weight", (96, 3, 4, 4), 48)))
    out.append((p + "patch_embed.projection.bias", init.bias(p + "patch_embed.projection.bias", (96,))))
    out += init.norm(p + "patch_embed.norm", 96)
    rel_index = relative_position_index(7)
    for s, (c, h, d) in enumerate(zip(SWIN_CHANNELS, SWIN_HEADS, SWIN_DEPTHS)):
        for b in range(d):
            q = f"{p}stages.{s}.blocks.{b}."
            out += init.norm(q + "norm1", c)
            out.append((q + "attn.w_msa.relative_position_bias_table",
                        randn(init.seed, q + "attn.w_msa.relative_position_bias_table", (169, h),
                              0.02 if init.mode == "baseline" else 0.5)))
            out.append((q + "attn.w_msa.relative_position_index", rel_index.copy()))
            out.append((q + "attn.w_msa.qkv.weight", init.weight(q + "attn.w_msa.qkv.weight", (3 * c, c), c)))
            out.append((q + "attn.w_msa.qkv.bias", init.bias(q + "attn.w_msa.qkv.bias", (3 * c,))))
            out.append((q + "attn.w_msa.proj.weight", init.weight(q + "attn.w_msa.proj.weight", (c, c), c)))
            out.append((q + "attn.w_msa.proj.bias", init.bias(q + "attn.w_msa.proj.bias", (c,))))
            out += init.norm(q + "norm2", c)
            out.append((q + "ffn.layers.0.0.weight", init.weight(q + "ffn.layers.0.0.weight", (4 * c, c), c)))
            out.append((q + "ffn.layers.0.0.bias", init.bias(q + "ffn.layers.0.0.bias", (4 * c,))))
            out.append((q + "ffn.layers.1.weight", init.weight(q + "ffn.layers.1.weight", (c, 4 * c), 4 * c)))
            out.append((q + "ffn.layers.1.bias", init.bias(q + "ffn.layers.1.bias", (c,))))
        if s < 3:
            q = f"{p}stages.{s}.downsample."
            out += init.norm(q + "norm", 4 * c)
            out.append((q + "reduction.weight", init.weight(q + "reduction.weight", (2 * c, 4 * c), 4 * c)))
    for i in range(1, 4):
        out += init.norm(f"{p}norm{i}", SWIN_CHANNELS[i])
    return out


def neck_tensors(init: _Init):
    out = []
    for level, cin in ((0, 448), (1, 1152)):
        for kind, ci, k in (("lateral_convs", cin, 1), ("fpn_convs", 256, 3)):
            q = f"neck.{kind}.{level}."
            out.append((q + "conv.weight", init.weight(q + "conv.weight", (256, ci, k, k), ci * k * k)))
            out += init.bn(q + "bn", 256)
    v = "vtransform."
    for conv, bn, co, ci, k in ((0, 1, 8, 1, 1), (3, 4, 32, 8, 5), (6, 7, 64, 32, 5)):
        q = f"{v}dtransform.{conv}."
        out.append((q + "weight", init.weight(q + "weight", (co, ci, k, k), ci * k * k)))
        out.append((q + "bias", init.bias(q + "bias", (co,))))
        out += init.bn(f"{v}dtransform.{bn}", co)
    for conv, bn, co, ci, k in ((0, 1, 256, 320, 3), (3, 4, 256, 256, 3)):
        q = f"{v}depthnet.{conv}."
        out.append((q + "weight", init.weight(q + "weight", (co, ci, k, k), ci * k * k)))
        out.append((q + "bias", init.bias(q + "bias", (co,))))
        out += init.bn(f"{v}depthnet.{bn}", co)
    out.append((v + "depthnet.6.weight", init.weight(v + "depthnet.6.weight", (198, 256, 1, 1), 256)))
    out.append((v + "depthnet.6.bias", init.bias(v + "depthnet.6.bias", (198,))))
    for conv, bn in ((0, 1), (3, 4), (6, 7)):
        q = f"{v}downsample.{conv}."
        out.append((q + "weight", init.weight(q + "weight", (80, 80, 3, 3), 720)))
        out += init.bn(f"{v}downsample.{bn}", 80)
    return out


def camera_branch_tensors(seed: int = 0, mode: str = "baseline", gain: float = 1.0,
                          offset: float = 0.0):
    init = _Init(seed, mode, gain, offset)
    return swin_tensors(init) + neck_tensors(init)


def write_camera_branch(path, seed: int = 0, mode: str = "baseline", gain: float = 1.0,
                        offset: float = 0.0) -> pathlib.Path:
    path = pathlib.Path(path)
    write_bfw(camera_branch_tensors(seed, mode, gain, offset), path)
    return path


def bev_stage_tensors(init: _Init):
    """Fuser, SECOND backbone + deblocks, TransFusion shared conv and heatmap
    head under the checkpoint's names and shapes (reference
    src/cuda_bev_stage.cu:239-255; ConvTranspose2d weights are [in, out, kH, kW])."""
    out = []

    def conv(name, shape, fan_in, bias=False):
        out.append((name + ".weight", init.weight(name + ".weight", shape, fan_in)))
        if bias:
            out.append((name + ".bias", init.bias(name + ".bias", shape[:1])))

    conv("fuser.conv.0", (256, 336, 3, 3), 336 * 9)
    out += init.bn("fuser.conv.1", 256)
    for b, (ch, first) in enumerate(((128, 256), (256, 128))):
        for l in range(6):
            ci = ch if l else first
            conv(f"backbone_2d.blocks.{b}.{3 * l + 1}", (ch, ci, 3, 3), ci * 9)
            out += init.bn(f"backbone_2d.blocks.{b}.{3 * l + 2}", ch)
    conv("backbone_2d.deblocks.0.0", (256, 128, 1, 1), 128)
    out += init.bn("backbone_2d.deblocks.0.1", 256)
    conv("backbone_2d.deblocks.1.0", (256, 256, 2, 2), 256)
    out += init.bn("backbone_2d.deblocks.1.1", 256)
    conv("dense_head.shared_conv", (128, 512, 3, 3), 512 * 9, bias=True)
    conv("dense_head.heatmap_head.0.conv", (128, 128, 3, 3), 128 * 9)
    out += init.bn("dense_head.heatmap_head.0.bn", 128)
    conv("dense_head.heatmap_head.1", (10, 128, 3, 3), 128 * 9, bias=True)
    return out


def transfusion_tensors(init: _Init):
    """TransFusion head under the checkpoint's names and shapes (reference
    src/transfusion_decoder.c:165-208): class encoding, one decoder layer
    (self / cross nn.MultiheadAttention, FFN, three LayerNorms, two position
    embedding heads) and six prediction heads.  The position heads' first
    conv sees cell coordinates up to the grid size, so it keeps std 0.02 in
    every mode."""
    out = []
    d = "dense_head.decoder."

    def w(name, shape, fan_in):
        out.append((name, init.weight(name, shape, fan_in)))

    def b(name, shape):
        out.append((name, init.bias(name, shape)))

    w("dense_head.class_encoding.weight", (128, 10, 1), 10)
    b("dense_head.class_encoding.bias", (128,))
    for attn in ("self_attn", "multihead_attn"):
        w(f"{d}{attn}.in_proj_weight", (384, 128), 128)
        b(f"{d}{attn}.in_proj_bias", (384,))
        w(f"{d}{attn}.out_proj.weight", (128, 128), 128)
        b(f"{d}{attn}.out_proj.bias", (128,))
    w(f"{d}linear1.weight", (256, 128), 128)
    b(f"{d}linear1.bias", (256,))
    w(f"{d}linear2.weight", (128, 256), 256)
    b(f"{d}linear2.bias", (128,))
    for i in (1, 2, 3):
        out += init.norm(f"{d}norm{i}", 128)
    for pos in ("self_posembed", "cross_posembed"):
        q = f"{d}{pos}.position_embedding_head."
        out.append((q + "0.weight", randn(init.seed, q + "0.weight", (128, 2, 1), 0.02)))
        b(q + "0.bias", (128,))
        out += init.bn(q + "1", 128)
        w(q + "3.weight", (128, 128, 1), 128)
        b(q + "3.bias", (128,))
    for head, ch in (("center", 2), ("height", 1), ("dim", 3), ("rot", 2), ("vel", 2),
                     ("heatmap", 10)):
        q = f"dense_head.prediction_head.{head}."
        w(q + "0.0.weight", (64, 128, 1), 128)
        out += init.bn(q + "0.1", 64)
        w(q + "1.weight", (ch, 64, 1), 64)
        b(q + "1.bias", (ch,))
    return out


def write_transfusion(path, seed: int = 0, mode: str = "baseline", gain: float = 1.0) -> pathlib.Path:
    path = pathlib.Path(path)
    write_bfw(transfusion_tensors(_Init(seed, mode, gain)), path)
    return path


def synthetic_transfusion_inputs(seed: int, height=180, width=180):
    """shared [1,128,H,W] ~N(0,1) and dense heatmap logits [1,10,H,W] ~N(-1, 1.5)."""
    return (randn(seed, "tf_shared", (1, 128, height, width)),
            randn(seed, "tf_heatmap", (1, 10, height, width), 1.5, -1.0))


def lidar_backbone_tensors(init: _Init):
    """SECOND sparse encoder under the checkpoint's names and shapes (reference
    src/lidar_backbone.c:94-133): weights [kd, kh, kw, Ci, Co] and a BN per
    conv (input SubM conv, four stages of two residual blocks, three strided
    convs, the (3,1,1) output conv)."""
    out = []
    p = "backbone_3d."

    def layer(w, bn, ci, co, k=(3, 3, 3)):
        out.append((w, init.weight(w, (*k, ci, co), k[0] * k[1] * k[2] * ci)))
        out.extend(init.bn(bn, co))

    layer(p + "conv_input.0.weight", p + "conv_input.1", 5, 16)
    ch = (16, 32, 64, 128)
    for s in range(4):
        for blk in range(2):
            for c in range(2):
                q = f"{p}conv{s + 1}.{blk + (1 if s else 0)}."
                layer(f"{q}conv{c + 1}.weight", f"{q}bn{c + 1}", ch[s], ch[s])
    for t in range(3):
        layer(f"{p}conv{t + 2}.0.0.weight", f"{p}conv{t + 2}.0.1", ch[t], ch[t + 1])
    layer(p + "conv_out.0.weight", p + "conv_out.1", 128, 128, (3, 1, 1))
    return out


def write_lidar_backbone(path, seed: int = 0, mode: str = "baseline",
                         gain: float = 1.0) -> pathlib.Path:
    path = pathlib.Path(path)
    write_bfw(lidar_backbone_tensors(_Init(seed, mode, gain)), path)
    return path


def synthetic_points(seed: int, count: int, clusters: int = 48, extent=54.0, z_range=(-5.0, 3.0),
                     sweeps: int = 1):
    """A LiDAR-like cloud [count, 5] (x, y, z, intensity, time): half on 32
    scan rings over a ground band, half in Gaussian clusters (objects) of
    0.2-1.5 m and, for a quarter of them, 2-5 cm, so voxels have occupied
    neighbours and some hold more than ten points.  With sweeps > 1 the ring
    returns repeat at `sweeps` azimuths 1 cm apart, as accumulated sweeps of
    a slowly moving sensor do.  A few points fall outside the range and a few
    are non-finite."""
    n_ring = count // 2
    n_obj = count - n_ring
    ring = randu(seed, "pts_ring", (n_ring,), 0, 32).astype(np.int64)
    radius = 2.0 + ring * (extent * 0.95 - 2.0) / 32.0
    theta = randu(seed, "pts_theta", (n_ring,), 0, 2 * np.pi)
    if sweeps > 1:
        base = np.arange(n_ring) // sweeps * sweeps
        ring, radius = ring[base], radius[base]
        theta = theta[base] + (np.arange(n_ring) % sweeps) * 0.01 / radius
    ground = np.stack([radius * np.cos(theta), radius * np.sin(theta),
                       randu(seed, "pts_ground", (n_ring,), -2.0, -1.7)], 1)
    centre = np.stack([randu(seed, "cl_x", (clusters,), -0.8 * extent, 0.8 * extent),
                       randu(seed, "cl_y", (clusters,), -0.8 * extent, 0.8 * extent),
                       randu(seed, "cl_z", (clusters,), -1.5, 1.0)], 1)
    size = randu(seed, "cl_s", (clusters,), 0.2, 1.5)
    size[: clusters // 4] = randu(seed, "cl_tight", (clusters // 4,), 0.02, 0.05)
    which = randu(seed, "pts_cl", (n_obj,), 0, clusters).astype(np.int64)
    obj = centre[which] + randn(seed, "pts_obj", (n_obj, 3)) * size[which, None]
    xyz = np.concatenate([ground, obj], 0)
    out = np.concatenate([xyz, randu(seed, "pts_int", (count, 1)),
                          randu(seed, "pts_t", (count, 1), 0.0, 0.5)], 1).astype(np.float32)
    # Shuffle so clusters interleave (first-encounter order matters).
    order = np.argsort(randu(seed, "pts_perm", (count,)), kind="stable")
    out = out[order]
    if count >= 20:
        out[3, 0] = 70.0                         # outside x
        out[7, 2] = z_range[1] + 1.0             # outside z
        out[11, 3] = np.nan                      # non-finite feature
    return np.ascontiguousarray(out)


def stress_points(count: int = 100000) -> np.ndarray:
    """The reference's LiDAR stress frame (tests/test_cuda_lidar.cu, its
    initialize_points): point i sits at the centre of voxel v = i // 2 of the
    production grid, x = v mod 1440, y = (v // 1440) mod 1440, z = hash(v) mod
    40 with hash(v) = (v * 2654435761) >> 16 (64-bit); intensity
    ((i mod 31) - 15) * 0.02, time ((i mod 17) - 8) * 0.01.  100k points give
    50k voxels, two points each, in a 1440 x 35 strip of columns."""
    i = np.arange(count, dtype=np.uint64)
    v = i // np.uint64(2)
    x = (v % np.uint64(1440)).astype(np.float32)
    y = ((v // np.uint64(1440)) % np.uint64(1440)).astype(np.float32)
    z = (((v * np.uint64(2654435761)) >> np.uint64(16)) % np.uint64(40)).astype(np.float32)
    f = np.float32
    out = np.stack([f(-54.0) + (x + f(0.5)) * f(0.075), f(-54.0) + (y + f(0.5)) * f(0.075),
                    f(-5.0) + (z + f(0.5)) * f(0.2),
                    ((i % np.uint64(31)).astype(np.int64) - 15).astype(np.float32) * f(0.02),
                    ((i % np.uint64(17)).astype(np.int64) - 8).astype(np.float32) * f(0.01)], 1)
    return np.ascontiguousarray(out, np.float32)


def write_bev_stage(path, seed: int = 0, mode: str = "baseline", gain: float = 1.0) -> pathlib.Path:
    path = pathlib.Path(path)
    write_bfw(bev_stage_tensors(_Init(seed, mode, gain)), path)
    return path


def full_model_tensors(seed: int = 0, mode: str = "fan_in", gain: float = 1.0):
    """Every tensor the frame runtime binds: Swin-T, camera neck (FPN, depth
    head, LSS downsample), SECOND encoder, BEV stage, TransFusion head and the
    LSS frustum vtransform.frustum [118,32,88,3]."""
    from . import frame_scene
    init = _Init(seed, mode, gain)
    return (swin_tensors(init) + neck_tensors(init) + lidar_backbone_tensors(init) +
            bev_stage_tensors(init) + transfusion_tensors(init) +
            [("vtransform.frustum", frame_scene.frustum())])


def write_full_model(path, seed: int = 0, mode: str = "fan_in", gain: float = 1.0) -> pathlib.Path:
    path = pathlib.Path(path)
    write_bfw(full_model_tensors(seed, mode, gain), path)
    return path


def synthetic_bev(seed: int, height=180, width=180, batches=1) -> np.ndarray:
    """Fused BEV input [B, 336, H, W] ~N(0,1): 80 image channels, then 256 lidar."""
    return randn(seed, "bev_input", (batches, 336, height, width))


# --------------------------------------------------------------------------
# Synthetic frame inputs
# --------------------------------------------------------------------------
IMAGENET_MEAN = np.array([0.485, 0.456, 0.406], dtype=np.float32)
IMAGENET_STD = np.array([0.229, 0.224, 0.225], dtype=np.float32)


def synthetic_images(seed: int, batches=6, height=256, width=704) -> np.ndarray:
    """U[0,1] pixels, ImageNet-normalised, NCHW float32."""
    img = randu(seed, "images", (batches, 3, height, width))
    return ((img - IMAGENET_MEAN[None, :, None, None]) / IMAGENET_STD[None, :, None, None]).astype(np.float32)


def synthetic_depth(seed: int, batches=6, height=256, width=704) -> np.ndarray:
    """Dense depth |N(0,1)|, [B,1,H,W] float32."""
    return np.abs(randn(seed, "dense_depth", (batches, 1, height, width)))
