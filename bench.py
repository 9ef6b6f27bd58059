#!/usr/bin/env python3
"""Benchmark: 6-camera 256x704 Swin-T + FPN + depth-head forward on one MI355X.

Workload (the config the metric is quoted on):
images [6,3,256,704] U[0,1] ImageNet-normalised and dense depth [6,1,256,704]
|N(0,1)|, 20 distinct frames (seeds 0-19) resident in HBM; random-init
weights ~N(0,0.02) under the checkpoint's tensor names (no network for the
real checkpoint).  One step = bf_cuda_swin_forward + bf_cuda_camera_neck_forward
(the reference runtime's camera calls, src/cuda_runtime.cu:74), replayed from
a HIP graph.  The timed region is bracketed by torch.cuda.synchronize().

Prints one JSON line with ms/frame, achieved TFLOP/s (304.4 GFLOP/frame), the
dominant kernel's roofline (timed live with HIP events) and the CPU baseline
(the reference's own CPU path, OpenMP, on this host's cores).

The same line carries an "lss" object: the lift-splat pooling that consumes
the depth head (include/bf_cuda.h), on the reference's production benchmark
inputs (tests/test_cuda_lss.cu:26-104: 6 cameras x 118 bins x 32x88, 80
channels, a 360x360 grid), timed as the reference reports it
(runs/rtx4060ti-2026-07-18/cuda_lss_intervals.txt): plan preparation from the
calibration plus one forward per frame, with the forward's roofline, its
measured HBM traffic and the reference's CPU pooling beside it.

A "bev_stage" object times the BEV stage after it (include/bf_cuda_bev.h,
the reference's 180x180 production shape, tests/test_cuda_bev_stage.cu:
94-118): 18 BN-folded convolutions on fp16 MFMA operands, with its roofline
(MFMA-bound) and the reference's CPU stage on the host.
"""

from __future__ import annotations

import argparse
import functools
import json
import os
import pathlib
import sys
import tempfile
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "bevfusion.c_amd"))

# Algorithmic work per frame (6 cameras): GEMM flops 2*M*N*K with window rows
# including padding tokens; see DESIGN.md "Measurement".
GFLOP_FRAME = 304.4
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-graph", action="store_true", help="launch eagerly instead of a HIP graph")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-cameras", type=int, default=6,
                   help="cameras in the CPU-baseline sample (6 = one full frame)")
    p.add_argument("--no-roofline", action="store_true", help="skip per-kernel timing")
    p.add_argument("--kernel-reps", type=int, default=20,
                   help="HIP-event timed launches per kernel in the roofline leg")
    p.add_argument("--kernels", default="",
                   help="comma-separated op names to time in the roofline leg (default: all)")
    p.add_argument("--no-traffic", action="store_true",
                   help="skip the rocprofv3 counter passes (MFMA utilisation and flops, "
                        "FETCH_SIZE / WRITE_SIZE) over every op")
    p.add_argument("--no-downsample", action="store_true", help="skip the downsample leg")
    p.add_argument("--no-config1", action="store_true", help="skip the config-1 linear leg")
    p.add_argument("--no-calibrate", action="store_true", help="skip the machine calibration leg")
    p.add_argument("--no-library", action="store_true",
                   help="skip the library-GEMM comparison leg (hipBLASLt on the Swin shapes)")
    p.add_argument("--pmc-child", default="",
                   help=argparse.SUPPRESS)  # internal: the program rocprofv3 profiles
    p.add_argument("--no-lss", action="store_true", help="skip the LSS pooling leg")
    p.add_argument("--no-bev", action="store_true", help="skip the BEV stage leg")
    p.add_argument("--no-tf", action="store_true", help="skip the TransFusion decoder leg")
    p.add_argument("--no-lidar", action="store_true", help="skip the LiDAR branch leg")
    p.add_argument("--no-runtime", action="store_true", help="skip the full-frame runtime leg")
    return p.parse_args()


def frame_flops(window_rows=True):
    """FLOPs of one frame, recomputed from the graph shapes.  With
    window_rows the QKV and proj GEMMs are charged at windows x 49 rows, as
    the reference computes them (padding tokens included: the
    reference-equivalent work); without, at the real token rows this build's
    kernels compute (the executed work)."""
    b = 6
    total = 0.0
    dims = [(64, 176), (32, 88), (16, 44), (8, 22)]
    for s, (c, d, heads) in enumerate(zip((96, 192, 384, 768), (2, 2, 6, 2), (3, 6, 12, 24))):
        h, w = dims[s]
        tok = b * h * w
        win_rows = b * ((h + 6) // 7) * ((w + 6) // 7) * 49
        rows = win_rows if window_rows else tok
        per_block = (2 * rows * c * 3 * c + 2 * rows * c * c                  # qkv, proj
                     + 2 * 2 * win_rows * 49 * c                              # QK^T, AV
                     + 2 * 2 * tok * c * 4 * c)                               # fc1, fc2
        total += d * per_block
        if s < 3:
            h2, w2 = dims[s + 1]
            total += 2 * b * h2 * w2 * 4 * c * 2 * c                         # merge
    total += 2 * b * 64 * 176 * 96 * 48                                      # patch embed
    h, w = 32, 88
    convs = [(16, 44, 256, 256, 3), (h, w, 256, 256, 3), (256, 704, 1, 8, 1), (64, 176, 8, 32, 5),
             (h, w, 32, 64, 5), (h, w, 320, 256, 3), (h, w, 256, 256, 3), (h, w, 256, 198, 1)]
    if window_rows:  # lateral 1x1 convs over the upsampled concat, as the reference runs them
        convs += [(16, 44, 1152, 256, 1), (h, w, 448, 256, 1)]
    else:  # lower halves at full resolution, upper halves at the upper level's
        convs += [(16, 44, 384, 256, 1), (8, 22, 768, 256, 1), (h, w, 192, 256, 1),
                  (16, 44, 256, 256, 1)]
    for oh, ow, ci, co, k in convs:
        total += 2 * b * oh * ow * co * ci * k * k
    return total


SWIN_STAGES = [(64, 176, 96, 3, 2), (32, 88, 192, 6, 2), (16, 44, 384, 12, 6),
               (8, 22, 768, 24, 2)]
# layer index: (name, output pixels M, Ci, Co, k, input bytes, output bytes
# per element).  Inputs are channels-last bf16 maps except dtransform.3,
# which reads the fp32 dense depth (its 8 input channels are computed from one
# value per pixel); depthnet.6 and the last downsample conv store fp32 NCHW.
DOWN_IN_HW = 360  # LSS BEV grid the downsample reads (reference production shape)
NECK_LAYERS = {
    0: ("fpn.lateral1", 6 * 16 * 44, 1152, 256, 1, 6 * 16 * 44 * 1152 * 2, 2),
    1: ("fpn.output1", 6 * 16 * 44, 256, 256, 3, 6 * 16 * 44 * 256 * 2, 2),
    2: ("fpn.lateral0", 6 * 32 * 88, 448, 256, 1, 6 * 32 * 88 * 448 * 2, 2),
    3: ("fpn.output0", 6 * 32 * 88, 256, 256, 3, 6 * 32 * 88 * 256 * 2, 2),
    4: ("depth.dtransform3", 6 * 64 * 176, 8, 32, 5, 6 * 256 * 704 * 4, 2),
    5: ("depth.dtransform6", 6 * 32 * 88, 32, 64, 5, 6 * 64 * 176 * 32 * 2, 2),
    6: ("depth.depthnet0", 6 * 32 * 88, 320, 256, 3, 6 * 32 * 88 * 320 * 2, 2),
    7: ("depth.depthnet3", 6 * 32 * 88, 256, 256, 3, 6 * 32 * 88 * 256 * 2, 2),
    8: ("depth.depthnet6", 6 * 32 * 88, 256, 198, 1, 6 * 32 * 88 * 256 * 2, 4),
    9: ("downsample.0", 360 * 360, 80, 80, 3, 360 * 360 * 80 * 2, 2),
    10: ("downsample.1", 180 * 180, 80, 80, 3, 360 * 360 * 80 * 2, 2),
    11: ("downsample.2", 180 * 180, 80, 80, 3, 180 * 180 * 80 * 2, 4),
}
IO_LAYERS = (4, 8, 11)  # timed on caller buffers (bfhip_camera_profile_layer_io)
# The lateral 1x1 convs over concat(lower, bilinear-up(upper)) run as two
# GEMMs (W_lower . lower, and W_upper . upper at the upper resolution, added
# upsampled in the first one's epilogue): layer -> (M, Cl, M_upper, Cu).  The
# forward runs the lower GEMM in one launch with a depth-encoder conv, so the
# op table times three launches: the upper products (hooks 0 and 2), and
# dtransform.3 / .6 each with its lateral's lower half (hooks 4 and 5).
LATERALS = {0: (6 * 16 * 44, 384, 6 * 8 * 22, 768), 2: (6 * 32 * 88, 192, 6 * 16 * 44, 256)}
PAIRED_LATERAL = {4: 0, 5: 2}  # depth-encoder layer -> the lateral whose lower half it shares a launch with


def swin_op_cost(stage, op, b=6):
    """Algorithmic FLOPs and HBM bytes of one launch of a Swin op: GEMM flops
    2*M*N*K over the tokens the kernel computes; bytes = every operand read
    once and every result written once at its stored width (bf16 activations
    and weights, fp32 residual stream)."""
    h, w, c, heads, _ = SWIN_STAGES[stage]
    t = b * h * w
    win = b * ((h + 6) // 7) * ((w + 6) // 7)
    st_b = t * (c // 64) * 8  # (mean, M2) per 64-channel group
    if op in ("ln1", "ln2"):
        return 8.0 * t * c, t * c * 4 + t * c * 2 + 8 * c
    if op == "qkv":  # LN1 folded: reads the fp16 residual copy and its statistics
        return 2.0 * t * c * 3 * c, t * c * 2 + st_b + 3 * c * c * 2 + t * 3 * c * 2
    if op == "attention":
        return 4.0 * win * 49 * 49 * c, t * 3 * c * 2 + t * c * 2 + heads * 49 * 49 * 4
    if op == "wmsa":  # fused QKV projection + attention: q, k, v stay on chip
        return (2.0 * t * c * 3 * c + 4.0 * win * 49 * 49 * c,
                t * c * 2 + 3 * c * c * 2 + t * c * 2 + heads * 49 * 49 * 4)
    if op == "proj":  # residual add; writes x, its fp16 copy and statistics
        return 2.0 * t * c * c, t * c * 2 + c * c * 2 + 2 * t * c * 4 + t * c * 2 + st_b
    if op == "fc1":  # LN2 folded
        return 2.0 * t * c * 4 * c, t * c * 2 + st_b + 4 * c * c * 2 + t * 4 * c * 2
    if op == "fc2":  # residual add (+ fp16 copy and statistics, except the last block)
        extra = 0 if stage == 3 else t * c * 2 + st_b
        return 2.0 * t * 4 * c * c, t * 4 * c * 2 + 4 * c * c * 2 + 2 * t * c * 4 + extra
    if op == "mlp":  # fused proj -> LN2 -> fc1 -> GELU -> fc2 -> residual (+ next LN1)
        return (2.0 * t * c * c + 4.0 * t * c * 4 * c,
                t * c * 4 * 2 + t * c * 2 * 2 + 9 * c * c * 2)
    if op == "merge":
        h2, w2 = SWIN_STAGES[stage + 1][:2]
        t2 = b * h2 * w2
        out = t2 * 2 * c * (4 + 2) + t2 * (2 * c // 64) * 8  # x, fp16 copy, statistics
        # LayerNorm folded: 2x2 tokens gathered from the fp16 copy and their
        # statistics (one 96-channel group per token at stage 0: st_b holds)
        return 2.0 * t2 * 4 * c * 2 * c, t * c * 2 + st_b + 8 * c * c * 2 + out
    raise ValueError(op)


def patch_embed_cost(b=6):
    """4x4/s4 conv 3 -> 96 + patch norm + LN1: fp32 images read, x (fp32) and
    xn (fp16) written."""
    t = b * 64 * 176
    return 2.0 * t * 96 * 48, b * 3 * 256 * 704 * 4 + t * 96 * (4 + 2) + 96 * 48 * 2


def out_norm_cost(stage, b=6):
    """Stage-output LayerNorm: x (fp32) and its (mean, M2) per 64 channels read,
    the NCHW fp32 output written."""
    h, w, c = SWIN_STAGES[stage][:3]
    t = b * h * w
    return 8.0 * t * c, t * c * 4 * 2 + t * (c // 64) * 8


def pack_cost(b=6):
    """Three Swin levels, NCHW fp32 read, channels-last fp16 written."""
    el = b * (192 * 32 * 88 + 384 * 16 * 44 + 768 * 8 * 22)
    return 0.0, el * (4 + 2)


def lateral_cost(layer, part):
    """The upper-level product ("upper": reads upper and W_upper, writes the
    fp32 product) or the lower half ("lower": reads lower, W_lower and the
    fp32 product, writes the output) of lateral `layer`."""
    m, cl, mu, cu = LATERALS[layer]
    if part == "upper":
        return 2.0 * 256 * mu * cu, mu * cu * 2 + 256 * cu * 2 + mu * 256 * 4
    return 2.0 * 256 * m * cl, m * cl * 2 + 256 * cl * 2 + mu * 256 * 4 + m * 256 * 2


def neck_layer_cost(layer):
    """Algorithmic FLOPs and HBM bytes of the launch(es) the op-table entry of
    neck `layer` runs (see PAIRED_LATERAL)."""
    if layer in LATERALS:
        return lateral_cost(layer, "upper")
    name, m, ci, co, k, in_bytes, out_el = NECK_LAYERS[layer]
    flops, nbytes = 2.0 * m * co * ci * k * k, in_bytes + co * ci * k * k * 2 + m * co * out_el
    if layer in PAIRED_LATERAL:
        lf, lb = lateral_cost(PAIRED_LATERAL[layer], "lower")
        flops, nbytes = flops + lf, nbytes + lb
    return flops, nbytes


def neck_io(dev):
    """Caller buffers the IO ops read or write: dense depth, logits, context,
    the downsample output, images (patch embedding) and the three Swin
    levels (output norms, level pack)."""
    import torch
    g = torch.Generator(device="cpu").manual_seed(0)
    return {"depth": torch.rand((6, 1, 256, 704), generator=g).to(dev),
            "logits": torch.empty((6, 118, 32, 88), device=dev),
            "ctx": torch.empty((6, 80, 32, 88), device=dev),
            "down": torch.empty((1, 80, DOWN_IN_HW // 2, DOWN_IN_HW // 2), device=dev),
            "images": torch.rand((6, 3, 256, 704), generator=g).to(dev),
            "levels": [torch.rand((6, c, h, w), generator=g).to(dev)
                       for c, h, w in ((192, 32, 88), (384, 16, 44), (768, 8, 22))]}


def roofline_entry(name, avg_s, per_frame, flops, nbytes):
    ai = flops / nbytes
    ridge = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    if ai >= ridge:
        achieved, peak, unit, bound = flops / avg_s / 1e12, PEAK_BF16_TFLOPS, "TFLOP/s", "mfma"
    else:
        achieved, peak, unit, bound = nbytes / avg_s / 1e9, PEAK_HBM_GBS, "GB/s", "hbm"
    return {"kernel": name, "bound": bound, "achieved": round(achieved, 1), "peak": peak,
            "unit": unit, "frac": round(achieved / peak, 4), "traffic": None,
            "avg_us": round(avg_s * 1e6, 2), "launches_per_frame": per_frame,
            "us_per_frame": round(avg_s * 1e6 * per_frame, 1),
            "flops_per_launch": flops, "bytes_per_launch": nbytes,
            "tflops": round(flops / avg_s / 1e12, 1), "gbs": round(nbytes / avg_s / 1e9, 1)}


def fused_stages(swin, stream):
    """Stages whose blocks run the fused MLP kernel (the library refuses
    their separate fc1 op)."""
    import bfhip
    out = []
    for st in range(4):
        try:
            swin.profile_op(st, 0, "mlp", stream)
            out.append(st)
        except bfhip.BfHipError:
            pass
    return out


def op_table(swin, neck, stream, io):
    """name -> (launch fn, launches per frame, (flops, bytes) per launch) for
    every op the forward launches (profiling hooks of include/bfhip_profile.h);
    `io` holds the caller buffers of neck_io()."""
    import bfhip
    table = {}
    fused = fused_stages(swin, stream)
    for st in range(4):
        depth = SWIN_STAGES[st][4]
        for op in ("ln1", "qkv", "attention", "wmsa", "proj", "ln2", "fc1", "fc2", "mlp"):
            try:  # ops a stage does not launch are refused by the library
                swin.profile_op(st, 0, op, stream)
            except bfhip.BfHipError:
                continue
            # LN1 runs once per stage when the previous block's fused MLP
            # already produced it.
            per_frame = 1 if (op == "ln1" and st in fused) else depth
            table[f"swin.s{st}.{op}"] = (lambda st=st, op=op: swin.profile_op(st, 0, op, stream),
                                         per_frame, swin_op_cost(st, op))
        if st == 0:
            table[f"swin.s{st}.merge"] = (lambda st=st: swin.profile_op(st, 0, "merge", stream),
                                          1, swin_op_cost(st, "merge"))
        elif st < 3:
            # The forward runs the merges after stages 1 and 2 in one launch
            # with that stage's output LayerNorm.
            mf, mb = swin_op_cost(st, "merge")
            lf, lb = out_norm_cost(st)
            table[f"swin.s{st}.merge_out_norm"] = (
                lambda st=st: swin.profile_io("merge_out_norm", st, out=io["levels"][st - 1],
                                              stream=stream), 1, (mf + lf, mb + lb))
    # The Swin launches outside the blocks and the neck's level pack.
    table["swin.patch_embed"] = (lambda: swin.profile_io("patch_embed", 0, images=io["images"],
                                                         stream=stream), 1, patch_embed_cost())
    table["swin.s3.out_norm"] = (
        lambda: swin.profile_io("out_norm", 3, out=io["levels"][2], stream=stream), 1,
        out_norm_cost(3))
    table["neck.pack"] = (lambda: neck.profile_pack(*io["levels"], stream=stream), 1, pack_cost())
    for layer, (name, *_rest) in NECK_LAYERS.items():
        if layer == 4:
            fn = lambda: neck.profile_layer_io(4, inp=io["depth"], stream=stream)
        elif layer == 8:
            fn = lambda: neck.profile_layer_io(8, out0=io["logits"], out1=io["ctx"], stream=stream)
        elif layer == 11:
            fn = lambda: neck.profile_layer_io(11, out0=io["down"], stream=stream)
        else:
            fn = lambda layer=layer: neck.profile_layer(layer, stream)
        if layer in LATERALS:
            name += "_upper"
        elif layer in PAIRED_LATERAL:
            name += "+" + NECK_LAYERS[PAIRED_LATERAL[layer]][0] + "_lower"
        table[f"neck.{name}"] = (fn, 1, neck_layer_cost(layer))
    return table


def time_kernels(swin, neck, stream, io, reps=20, only=()):
    """Time single ops of the path with HIP events on the stream they are
    launched on; returns roofline entries sorted by time per frame.  The
    downsample layers run once per LSS output, not per camera frame: they are
    timed here (and reported under "downsample") but kept out of the frame's
    ranking."""
    import torch
    out = []
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for name, (fn, per_frame, (flops, nbytes)) in op_table(swin, neck, stream, io).items():
        if only and name not in only:
            continue
        for _ in range(3):
            fn()
        start.record(stream)
        for _ in range(reps):
            fn()
        stop.record(stream)
        stop.synchronize()
        avg_s = start.elapsed_time(stop) / 1e3 / reps
        out.append(roofline_entry(name, avg_s, per_frame, flops, nbytes))
    out.sort(key=lambda e: -e["us_per_frame"])
    return out


# HBM traffic of one op, from two rocprofv3 counter passes over a child run of
# this script (--pmc-child): FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of
# the op's kernels, each scaled by what the same counter reads for a plain
# device copy of known size in the same run.
PMC_OP_REPS, PMC_COPY_REPS, PMC_COPY_BYTES = 23, 29, 64 << 20


ALL_OPS = "@all"        # --pmc-child: every op of the table, separated by marker launches
ALL_OP_REPS = 5
MARKER_KERNEL = "calib_empty_kernel"


def _camera_contexts(dev):
    """The bench's Swin and camera-neck contexts at 6 x 256 x 704 on a
    synthetic checkpoint, after one forward (so every scratch buffer holds
    realistic activations)."""
    import torch
    import bfhip
    from bfhip import bfw
    tmp = pathlib.Path(tempfile.mkdtemp(prefix="pmc_"))
    model_path = bfw.write_camera_branch(tmp / "camera_branch.bfw", seed=0, mode="baseline")
    with bfhip.Model(model_path) as m:
        swin = bfhip.Swin(m, 6, 256, 704)
        neck = bfhip.CameraNeck(m, 6, 32, 88, DOWN_IN_HW, DOWN_IN_HW)
    img = torch.from_numpy(bfw.synthetic_images(0, 6, 256, 704)).to(dev)
    dep = torch.from_numpy(bfw.synthetic_depth(0, 6, 256, 704)).to(dev)
    return swin, neck, img, dep


def pmc_child(op):
    """Body of the profiled child: a 64 MiB device-to-device copy
    PMC_COPY_REPS times (the calibration kernel), then the op PMC_OP_REPS
    times; every dispatch after the last copy belongs to the op.  With
    op == ALL_OPS, every op of op_table() runs ALL_OP_REPS times instead,
    each preceded by one empty marker kernel, and one marker closes the run."""
    import torch
    import bfhip
    dev = torch.device("cuda:0")
    if op == LSS_OP:
        plan, fwd = lss_setup(dev)
        src = torch.zeros(PMC_COPY_BYTES // 4, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(PMC_COPY_REPS):
            dst.copy_(src)
        torch.cuda.synchronize()
        for _ in range(PMC_OP_REPS):
            fwd()
        torch.cuda.synchronize()
        plan.close()
        return
    swin, neck, img, dep = _camera_contexts(dev)
    io = neck_io(dev)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        outs = swin.forward(img, stream=stream)
        neck.neck_forward(*outs, dep, stream=stream)
        neck.downsample_forward(torch.rand((1, 80, DOWN_IN_HW, DOWN_IN_HW), device=dev),
                                stream=stream)
        table = op_table(swin, neck, stream, io)
        src = torch.zeros(PMC_COPY_BYTES // 4, device=dev)
        dst = torch.empty_like(src)
        stream.synchronize()
        for _ in range(PMC_COPY_REPS):
            dst.copy_(src)
        stream.synchronize()
        if op == ALL_OPS:
            for name, (fn, *_rest) in table.items():
                bfhip.calibrate("empty", 1, stream=stream)
                for _ in range(ALL_OP_REPS):
                    fn()
                stream.synchronize()
            bfhip.calibrate("empty", 1, stream=stream)
        else:
            for _ in range(PMC_OP_REPS):
                table[op][0]()
        stream.synchronize()


def _pmc_pass(counters, child_op, timeout_s):
    """One rocprofv3 counter pass over `bench.py --pmc-child child_op`:
    returns (dispatch rows sorted by id as dicts {id, kernel, grid, values},
    None) or (None, reason)."""
    import csv
    import shutil
    import subprocess
    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(prof):
        return None, "rocprofv3 not found"
    out = pathlib.Path(tempfile.mkdtemp(prefix="pmc_", dir="/tmp"))
    cmd = ["timeout", "-s", "KILL", str(timeout_s), prof, "--pmc", *counters,
           "--output-format", "csv", "-d", str(out), "-o", "p", "--",
           os.path.realpath(sys.executable), str(ROOT / "bench.py"), "--pmc-child", child_op]
    env = dict(os.environ, TMPDIR="/tmp")
    proc = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True)
    files = list(out.rglob("*counter_collection.csv"))
    if not files:
        tail = (proc.stderr or proc.stdout).strip().splitlines()[-3:]
        return None, f"{' '.join(counters)}: no counters (exit {proc.returncode}): {' | '.join(tail)}"
    rows = {}
    for r in csv.DictReader(open(files[0])):
        d = rows.setdefault(int(r["Dispatch_Id"]), {"id": int(r["Dispatch_Id"]),
                                                     "kernel": r["Kernel_Name"],
                                                     "grid": r["Grid_Size"], "values": {}})
        d["values"][r["Counter_Name"]] = d["values"].get(r["Counter_Name"], 0.0) + \
            float(r["Counter_Value"])
    shutil.rmtree(out, ignore_errors=True)
    return [rows[k] for k in sorted(rows)], None


def _copy_scale(rows, counter):
    """(index of the first dispatch after the calibration copies, bytes per
    counter unit) from the PMC_COPY_REPS copies at the start of a pass."""
    import statistics
    groups = {}
    for i, r in enumerate(rows):
        groups.setdefault((r["kernel"], r["grid"]), []).append(i)
    copy = [g for g in groups.values() if len(g) == PMC_COPY_REPS]
    if len(copy) != 1:
        return None, None
    kib = statistics.median(rows[i]["values"][counter] for i in copy[0])
    return max(copy[0]) + 1, PMC_COPY_BYTES / (kib * 1024)


def measure_op_counters(names, timeout_s=240):
    """Per-launch counters of every op in `names` (op_table order) from three
    rocprofv3 passes over one child run each: MFMA (MfmaUtil, MfmaFlopsBF16,
    MfmaFlopsF16) and HBM traffic (FETCH_SIZE, WRITE_SIZE; KiB scaled by a
    64 MiB copy).  Returns ({name: {...}}, [errors])."""
    passes = [("mfma", ["MfmaUtil", "MfmaFlopsBF16", "MfmaFlopsF16"]),
              ("fetch", ["FETCH_SIZE"]), ("write", ["WRITE_SIZE"])]
    result = {n: {} for n in names}
    errors = []
    for kind, counters in passes:
        rows, why = _pmc_pass(counters, ALL_OPS, timeout_s)
        if rows is None:
            errors.append(why)
            continue
        start, scale = _copy_scale(rows, counters[0]) if kind != "mfma" else (0, 1.0)
        if start is None:
            errors.append(f"{kind}: calibration copy not identified")
            continue
        marks = [i for i in range(start, len(rows)) if MARKER_KERNEL in rows[i]["kernel"]]
        if len(marks) != len(names) + 1:
            errors.append(f"{kind}: {len(marks)} markers for {len(names)} ops")
            continue
        for k, name in enumerate(names):
            seg = rows[marks[k] + 1:marks[k + 1]]
            if not seg or len(seg) % ALL_OP_REPS:
                errors.append(f"{kind}: {name} has {len(seg)} dispatches")
                continue
            tot = {c: sum(r["values"].get(c, 0.0) for r in seg) for c in counters}
            e = result[name]
            if kind == "mfma":
                # An op of several kernels (merge: LayerNorm + GEMM) reports
                # the utilisation of its MFMA kernel, the one with most flops.
                per = len(seg) // ALL_OP_REPS
                flops = lambda r: r["values"].get("MfmaFlopsBF16", 0.0) + \
                    r["values"].get("MfmaFlopsF16", 0.0)
                main = max(range(per), key=lambda j: sum(flops(r) for r in seg[j::per]))
                util = [r["values"].get("MfmaUtil", 0.0) for r in seg[main::per]]
                e["mfma_util_pct"] = round(sum(util) / len(util), 2)
                e["mfma_flops"] = (tot["MfmaFlopsBF16"] + tot["MfmaFlopsF16"]) / ALL_OP_REPS
                e["kernels_per_launch"] = per
            else:
                e[f"{kind}_bytes"] = round(tot[counters[0]] * 1024 * scale / ALL_OP_REPS)
                e[f"{kind}_scale"] = round(scale, 4)
    return result, errors


def measure_traffic(op, timeout_s=120):
    """Scaled HBM bytes per launch of `op`, or (None, reason)."""
    import csv
    import shutil
    import statistics
    import subprocess
    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(prof):
        return None, "rocprofv3 not found"
    per = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        out = pathlib.Path(tempfile.mkdtemp(prefix=f"pmc_{counter}_", dir="/tmp"))
        cmd = ["timeout", "-s", "KILL", str(timeout_s), prof, "--pmc", counter,
               "--output-format", "csv", "-d", str(out), "-o", "p", "--",
               os.path.realpath(sys.executable), str(ROOT / "bench.py"), "--pmc-child", op]
        env = dict(os.environ, TMPDIR="/tmp")
        proc = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True)
        files = list(out.rglob("*counter_collection.csv"))
        if not files:
            return None, f"{counter} pass produced no counters (exit {proc.returncode})"
        rows = [r for r in csv.DictReader(open(files[0])) if r.get("Counter_Name") == counter]
        rows.sort(key=lambda r: int(r["Dispatch_Id"]))
        groups = {}
        for r in rows:
            groups.setdefault((r["Kernel_Name"], r["Grid_Size"]), []).append(r)
        copy = [g for g in groups.values() if len(g) == PMC_COPY_REPS]
        if len(copy) != 1:
            return None, f"{counter}: calibration copy not identified in the counter dump"
        last_copy = max(int(r["Dispatch_Id"]) for r in copy[0])
        after = [r for r in rows if int(r["Dispatch_Id"]) > last_copy]
        if not after or len(after) % PMC_OP_REPS:
            return None, f"{counter}: {len(after)} op dispatches, expected a multiple of {PMC_OP_REPS}"
        op_kib = sum(float(r["Counter_Value"]) for r in after) / PMC_OP_REPS
        copy_kib = statistics.median(float(r["Counter_Value"]) for r in copy[0])
        per[counter] = (op_kib, (PMC_COPY_BYTES / 1024) / copy_kib)
    fetch = per["FETCH_SIZE"][0] * per["FETCH_SIZE"][1] * 1024
    write = per["WRITE_SIZE"][0] * per["WRITE_SIZE"][1] * 1024
    return {"bytes": round(fetch + write), "fetch_bytes": round(fetch), "write_bytes": round(write),
            "fetch_kib_raw": round(per["FETCH_SIZE"][0], 1), "write_kib_raw": round(per["WRITE_SIZE"][0], 1),
            "fetch_scale": round(per["FETCH_SIZE"][1], 4), "write_scale": round(per["WRITE_SIZE"][1], 4),
            "calibration": f"{PMC_COPY_BYTES >> 20} MiB device copy"}, None


# Post-LSS downsample (three 3x3 80->80 convs from 360x360 plus the x/y
# transpose), reference RTX 4060 Ti warm time (runs/rtx4060ti-2026-07-18/
# cuda_camera_slice.txt:13; benchmark.csv:16; entry src/cuda_camera.cu:409-422).
DOWN_REFERENCE_MS = 2.397


def downsample_leg(neck, dev, stream, reps, kernels):
    """bf_cuda_camera_downsample_forward on the reference's production BEV
    (1 x 80 x 360 x 360 fp32 in, 1 x 80 x 180 x 180 out), replayed from a HIP
    graph and timed with HIP events; the per-layer entries come from the
    roofline leg's `kernels` list."""
    import torch
    hw = DOWN_IN_HW
    g = torch.Generator(device="cpu").manual_seed(7)
    bev = torch.rand((1, 80, hw, hw), generator=g).to(dev)
    out = torch.empty((1, 80, hw // 2, hw // 2), device=dev)
    flops = sum(neck_layer_cost(l)[0] for l in (9, 10, 11))
    nbytes = bev.numel() * 4 + out.numel() * 4 + 3 * 80 * 80 * 9 * 2
    with torch.cuda.stream(stream):
        neck.downsample_forward(bev, out, stream=stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            neck.downsample_forward(bev, out, stream=stream)
        for _ in range(3):
            graph.replay()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps):
            graph.replay()
        stop.record(stream)
        stop.synchronize()
    ms = start.elapsed_time(stop) / reps
    roof = roofline_entry("downsample forward (pack + 3 convs + transposed store)", ms / 1e3, 1,
                          flops, nbytes)
    layers = [k for k in kernels if k["kernel"].startswith("neck.downsample")]
    return {"workload": "post-LSS downsample, reference production shape: 1 x 80 x 360 x 360 fp32 "
                        "-> 3x3 s1 -> 3x3 s2 -> 3x3 s1 (BN-folded, ReLU) -> x/y-transposed "
                        "1 x 80 x 180 x 180",
            "ms": round(ms, 4), "gflop": round(flops / 1e9, 2),
            "tflops": round(flops / ms / 1e9, 1),
            "reference_rtx4060ti_ms": DOWN_REFERENCE_MS,
            "speedup_vs_reference": round(DOWN_REFERENCE_MS / ms, 1),
            "roofline": {k: roof[k] for k in ("kernel", "bound", "achieved", "peak", "unit", "frac",
                                               "traffic")},
            "layers": layers}


# one fp32 linear as in Swin-T stage-1 QKV, X[11264 x 96]
# W[288 x 96] + bias, N(0,1)/sqrt(96), seed 0 (reference CPU kernels_ref.c:
# 292-339 and its dispatch test tests/test_cpu_dispatch.c:25-70; GPU entry
# point bf_cuda_gemm_f32, src/cuda_ops.cu:188-208).
CONFIG1 = (11264, 96, 288)


def config1_inputs():
    import numpy as np
    m, k, n = CONFIG1
    rng = np.random.default_rng(0)
    sc = 1.0 / np.sqrt(k)
    x = (rng.standard_normal((m, k)) * sc).astype(np.float32)
    w = (rng.standard_normal((n, k)) * sc).astype(np.float32)
    b = (rng.standard_normal(n) * sc).astype(np.float32)
    return x, w, b


def config1_leg(dev, reps, with_cpu):
    """bf_cuda_gemm_f32 at config 1 (HIP events, eager launches on one
    stream); the CPU side times the reference's linear (its OpenMP split and
    its scalar kernel) as a median of >= 20 calls."""
    import statistics
    import torch
    import bfhip
    m, k, n = CONFIG1
    x, w, b = config1_inputs()
    flops = 2.0 * m * n * k
    nbytes = (x.size + w.size + b.size + m * n) * 4
    xd, wd, bd = (torch.from_numpy(a).to(dev) for a in (x, w, b))
    yd = torch.empty((m, n), device=dev)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for _ in range(5):
            bfhip.gemm_f32(xd, wd, bd, out=yd, stream=stream)
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps):
            bfhip.gemm_f32(xd, wd, bd, out=yd, stream=stream)
        stop.record(stream)
        stop.synchronize()
    avg_s = start.elapsed_time(stop) / 1e3 / reps
    roof = roofline_entry("bf_cuda_gemm_f32 11264x96 -> 288 (fp32 in/out)", avg_s, 1, flops, nbytes)
    out = {"workload": "BASELINE config 1: fp32 linear X[11264x96] W[288x96]^T + b, "
                       "N(0,1)/sqrt(96), seed 0",
           "gpu": {"us": round(avg_s * 1e6, 2), "gflop_per_s": round(flops / avg_s / 1e9, 1),
                   "roofline": {kk: roof[kk] for kk in ("bound", "achieved", "peak", "unit",
                                                        "frac")}}}
    if with_cpu:
        import oracle
        flavour = "ref_o3" if oracle.available("ref_o3") else "port"
        o = oracle.Oracle(flavour)
        cpu = {}
        for label, scalar in (("optimized", False), ("scalar", True)):
            times = []
            for _ in range(21):
                t0 = time.perf_counter()
                o.linear(x, w, b, scalar=scalar)
                times.append(time.perf_counter() - t0)
            med = statistics.median(times[1:])
            cpu[label] = {"ms": round(med * 1e3, 3), "gflop_per_s": round(flops / med / 1e9, 2),
                          "reps": len(times) - 1}
        cpu.update(_cpu_host(), kind="reference" if flavour == "ref_o3" else "port",
                   backend=o.backend())
        out["cpu"] = cpu
    return out


def calibrate_leg(dev):
    """Machine rates behind the roofline discussion, from the calibration
    kernels of include/bfhip_profile.h: launch cost (eager and inside a HIP
    graph), sustained bf16 MFMA rate of the 16x16x32 and 32x32x16 shapes, LDS
    read bandwidth and device copy bandwidth."""
    import torch
    import bfhip
    stream = torch.cuda.Stream()
    ev = lambda: torch.cuda.Event(enable_timing=True)

    def timed(fn, reps):
        fn()
        start, stop = ev(), ev()
        start.record(stream)
        for _ in range(reps):
            fn()
        stop.record(stream)
        stop.synchronize()
        return start.elapsed_time(stop) / 1e3 / reps

    out = {}
    with torch.cuda.stream(stream):
        launches = 200
        out["launch_us_eager"] = round(1e6 * timed(lambda: bfhip.calibrate("empty", 1, stream=stream),
                                                   launches), 3)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(launches):
                bfhip.calibrate("empty", 1, stream=stream)
        out["launch_us_graph"] = round(1e6 * timed(graph.replay, 5) / launches, 3)
        sink = torch.empty(1024 * 256, device=dev)
        grid, iters = 512, 2000
        t = timed(lambda: bfhip.calibrate("mfma16", grid, iters, dst=sink, stream=stream), 5)
        out["mfma16x16x32_bf16_tflops"] = round(grid * 4 * iters * 8 * 16384 / t / 1e12, 1)
        t = timed(lambda: bfhip.calibrate("mfma32", grid, iters, dst=sink, stream=stream), 5)
        out["mfma32x32x16_bf16_tflops"] = round(grid * 4 * iters * 8 * 32768 / t / 1e12, 1)
        lgrid, liters = 1024, 4000
        t = timed(lambda: bfhip.calibrate("lds", lgrid, liters, dst=sink, stream=stream), 5)
        lds = lgrid * 256 * liters * 16 / t
        out["lds_read_tb_s"] = round(lds / 1e12, 2)
        out["lds_read_b_per_clk_per_cu_at_2_4ghz"] = round(lds / 256 / 2.4e9, 1)
        # MFMA fed from LDS as in the GEMM cores: 4 workgroups of 8 waves per
        # CU; 64 x 64 wave tiles with random or constant fp16 operands, and
        # 32 x 32 wave tiles (LDS-heavy) for the fragment-read bandwidth.
        mgrid, miters = 1024, 2000
        for kind, fm, key, lds_key in (
                ("mfma_lds", 4, "mfma16_lds_random_tflops", None),
                ("mfma_lds_flat", 4, "mfma16_lds_constant_tflops", None),
                ("mfma_lds_narrow", 2, "mfma16_lds_random_32x32_tflops", "lds_fragment_read"),
                ("mfma_lds_narrow_flat", 2, "mfma16_lds_constant_32x32_tflops",
                 "lds_fragment_read_constant")):
            t = timed(lambda kind=kind: bfhip.calibrate(kind, mgrid, miters, dst=sink, stream=stream), 5)
            waves = mgrid * 8 * miters
            out[key] = round(waves * 2 * fm * fm * 16384 / t / 1e12, 1)
            if lds_key:
                lds_f = waves * 2 * (2 * fm) * 1024 / t
                out[lds_key + "_tb_s"] = round(lds_f / 1e12, 1)
                out[lds_key + "_b_per_clk_per_cu_at_2_4ghz"] = round(lds_f / 256 / 2.4e9, 1)
        src = torch.zeros(256 << 20, device=dev)  # 1 GiB
        dst = torch.empty_like(src)
        t = timed(lambda: bfhip.calibrate("copy", 4096, src=src, dst=dst, stream=stream), 5)
        out["copy_gb_s"] = round(2 * src.numel() * 4 / t / 1e9, 1)
        del src, dst
    out["note"] = ("MFMA kernels: 2 workgroups of 4 waves per CU, 8 independent accumulator "
                   "chains per wave, register operands; LDS: 4 workgroups per CU, conflict-free "
                   "16-byte reads issued 8 at a time with a VALU add per read; mfma16_lds_*: 4 "
                   "workgroups of 8 waves per CU reading fp16 fragments from LDS each step as the "
                   "GEMM cores do (random operands draw more power, hence a lower clock, than "
                   "constant ones); copy: 1 GiB float4, read + write bytes")
    return out


def library_gemm_leg(dev, kernels, reps=50):
    """The Swin-T linear shapes at 6x256x704 as plain library GEMMs, for
    comparison with this library's ops: torch.nn.functional.linear in bf16
    (X [M, K] and W [N, K] row-major, no bias, no epilogue), which ROCm's
    PyTorch hands to hipBLASLt when that is the preferred BLAS library.  Each
    shape runs `reps` times in one captured HIP graph, timed with HIP events
    on the capture stream.  Beside each shape: this library's op of the same
    stage and shape from the roofline leg (fused epilogue included: folded
    LayerNorm, bias, GELU, residual add and row statistics), where the
    forward launches it as a separate op."""
    import torch
    import torch.nn.functional as F
    ours = {e["kernel"]: e["avg_us"] for e in kernels}
    try:
        torch.backends.cuda.preferred_blas_library("hipblaslt")
    except (RuntimeError, AttributeError):
        pass
    # torch names the Lt backend after CUDA's; on ROCm it is hipBLASLt.
    backend = str(torch.backends.cuda.preferred_blas_library()).split(".")[-1]
    library = {"Cublaslt": "hipBLASLt", "Cublas": "rocBLAS", "Ck": "composable_kernel"}.get(
        backend, backend)
    stream = torch.cuda.Stream()
    ev = lambda: torch.cuda.Event(enable_timing=True)
    rows = []
    with torch.cuda.stream(stream):
        for st, (h, w, c, _heads, _depth) in enumerate(SWIN_STAGES):
            m = 6 * h * w
            for op, n, k in (("qkv", 3 * c, c), ("proj", c, c), ("fc1", 4 * c, c),
                             ("fc2", c, 4 * c)):
                gen = torch.Generator(device=dev).manual_seed(1000 * st + n + k)
                x = torch.randn(m, k, device=dev, dtype=torch.bfloat16, generator=gen)
                wt = (0.02 * torch.randn(n, k, device=dev, generator=gen)).to(torch.bfloat16)
                y = F.linear(x, wt)
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=stream):
                    for _ in range(reps):
                        y = F.linear(x, wt)
                g.replay()
                start, stop = ev(), ev()
                start.record(stream)
                for _ in range(3):
                    g.replay()
                stop.record(stream)
                stop.synchronize()
                us = start.elapsed_time(stop) * 1e3 / (3 * reps)
                name = f"swin.s{st}.{op}"
                row = {"op": name, "m": m, "n": n, "k": k, "library_us": round(us, 2),
                       "library_tflops": round(2.0 * m * n * k / us / 1e6, 1)}
                if name in ours:
                    row["ours_us"] = ours[name]
                rows.append(row)
                del g, x, wt, y
    return {"library": library, "dtype": "bf16", "reps_per_graph": reps, "rows": rows,
            "note": "library: torch.nn.functional.linear, no epilogue; ours: the op's own "
                    "kernel from the roofline leg, with its fused epilogue"}


LSS_OP = "lss_forward"
# Reference timings of the same benchmark on an RTX 4060 Ti
# (runs/rtx4060ti-2026-07-18/cuda_lss_intervals.txt:14-16).
LSS_REFERENCE_MS = {"forward": 1.389, "prepare_calibration": 0.363, "total": 1.752}


def lss_setup(dev, stream=None):
    """Production LSS inputs resident on the GPU and a prepared plan; returns
    (plan, forward callable)."""
    import torch
    import bfhip
    from bfhip import lss_scene
    sc = lss_scene.production()
    d = sc["desc"]
    desc = bfhip.lss_desc(d["batches"], d["cameras"], d["depth_bins"], d["height"], d["width"],
                          d["channels"], d["minimum"], d["step"], d["cells"])
    put = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    logits, ctx, frustum = put(sc["depth_logits"]), put(sc["context"]), put(sc["frustum"])
    cal = [put(sc[k]) for k in lss_scene.CALIBRATION_KEYS]
    bev = torch.empty((1, d["channels"] * d["cells"][2], d["cells"][0], d["cells"][1]),
                      device=dev)
    plan = bfhip.LssPlan(desc)
    plan.prepare_calibration(frustum, *cal, stream=stream)
    plan.inputs = (logits, ctx, frustum, cal, bev, sc)
    return plan, lambda: plan.forward(logits, ctx, out=bev, stream=stream)


def lss_leg(dev, reps, traffic):
    """LSS pooling on the reference's production inputs (see the module
    docstring): ms for prepare + forward, forward, prepare; the forward's
    roofline against HBM; the reference CPU pooling on the host."""
    import torch
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        plan, fwd = lss_setup(dev, stream)
        logits, ctx, frustum, cal, bev, sc = plan.inputs

        def prep():
            plan.prepare_calibration(frustum, *cal, stream=stream)

        def timed(fn):
            for _ in range(3):
                fn()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for _ in range(reps):
                fn()
            b.record(stream)
            b.synchronize()
            return a.elapsed_time(b) / reps

        ms_fwd = timed(fwd)
        ms_prep = timed(prep)
        ms_total = timed(lambda: (prep(), fwd()))
        stream.synchronize()
    d = sc["desc"]
    samples = d["cameras"] * d["depth_bins"] * d["height"] * d["width"]
    # compulsory HBM bytes of one forward: logits + context in, BEV out (fp32)
    nbytes = 4 * (samples + d["cameras"] * d["channels"] * d["height"] * d["width"]
                  + d["channels"] * d["cells"][0] * d["cells"][1] * d["cells"][2])
    gbs = nbytes / (ms_fwd * 1e-3) / 1e9
    roof = {"kernel": "lss plan forward (softmax stats + context rows + pool + combine)",
            "bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
            "algorithmic_bytes": nbytes, "avg_us": round(ms_fwd * 1e3, 2),
            "note": "the pool gathers one 320 B context row per sample (2.0 M samples) "
                    "through L2; compulsory HBM bytes understate its memory work"}
    if traffic:
        t, why = measure_traffic(LSS_OP)
        if t:
            roof["traffic"] = t["bytes"]
            roof["traffic_detail"] = t
        else:
            roof["traffic_error"] = why
    out = {"workload": "reference production LSS benchmark (tests/test_cuda_lss.cu:26-104): "
                       "1 batch x 6 cameras x 118 depth bins x 32x88, 80 channels, "
                       "360x360x1 grid of 0.3 m; plan prepared from calibration each frame",
           "ms_per_frame": round(ms_total, 4), "ms_forward": round(ms_fwd, 4),
           "ms_prepare_calibration": round(ms_prep, 4),
           "reference_rtx4060ti_ms": LSS_REFERENCE_MS,
           "plan_resident_mib": round(plan.resident_bytes() / 2**20, 2),
           "roofline": roof}
    plan.close()
    return out, sc


def lss_cpu_baseline(sc):
    """The reference's CPU geometry + fused lift-pool (oracle/_ref, src/lss.c)
    on the full production frame, single-threaded (lss.c has no OpenMP)."""
    import oracle
    kind = "reference" if oracle.available("ref_o3") else "port"
    o = oracle.Oracle("ref_o3" if kind == "reference" else "port")
    d = sc["desc"]
    desc = oracle.lss_desc(d["batches"], d["cameras"], d["depth_bins"], d["height"],
                           d["width"], d["channels"], d["minimum"], d["step"], d["cells"])
    t0 = time.perf_counter()
    g = o.lss_geometry(sc["frustum"], sc["camera_rotation"], sc["camera_translation"],
                       sc["intrinsics"], sc["post_rotation"], sc["post_translation"],
                       sc["extra_rotation"], sc["extra_translation"])
    t1 = time.perf_counter()
    o.lss_lift_pool(sc["depth_logits"], sc["context"], g, desc)
    t2 = time.perf_counter()
    return {"value": round((t2 - t0) * 1e3, 1), "unit": "ms/frame", "cores": 1, "kind": kind,
            "sample": f"one full production frame: geometry {1e3 * (t1 - t0):.0f} ms + "
                      f"lift-pool {1e3 * (t2 - t1):.0f} ms",
            "cpu_model": _cpu_model()}


BEV_HW = 180
# Reference BEV stage on the RTX 4060 Ti (cuDNN, fp32 FMA math;
# runs/rtx4060ti-2026-07-18/benchmark.csv:4) and its CPU stage (README.md:247).
BEV_REFERENCE = {"gpu_ms": 19.6, "cpu_ms": 6110.0}


def bev_layers(h=BEV_HW, w=BEV_HW):
    """(name, M, N, K) of every GEMM of the stage (reference layer table,
    cuda_bev_stage.cu:239-255)."""
    hw, hw2 = h * w, (h // 2) * (w // 2)
    out = [("fuser", hw, 256, 336 * 9)]
    out += [(f"block0.{l}", hw, 128, (128 if l else 256) * 9) for l in range(6)]
    out += [("deblock0", hw, 256, 128)]
    out += [(f"block1.{l}", hw2, 256, (256 if l else 128) * 9) for l in range(6)]
    out += [("deblock1", hw2, 1024, 256), ("shared", hw, 128, 512 * 9),
            ("heatmap_mid", hw, 128, 128 * 9), ("heatmap_out", hw, 10, 128 * 9)]
    return out


def bev_leg(dev, reps, seed=0):
    """BEV stage at 180x180: ms per forward, TFLOP/s, MFMA roofline."""
    import torch
    import bfhip
    from bfhip import bfw
    tmp = pathlib.Path(tempfile.mkdtemp(prefix="bev_"))
    path = bfw.write_bev_stage(tmp / "bev.bfw", seed=seed, mode="baseline")
    x = torch.from_numpy(bfw.synthetic_bev(seed, BEV_HW, BEV_HW)).to(dev)
    stream = torch.cuda.Stream()
    with bfhip.Model(path) as m:
        stage = bfhip.BevStage(m, BEV_HW, BEV_HW)
    with torch.cuda.stream(stream):
        outs = stage.forward(x, stream=stream)
        for _ in range(3):
            stage.forward(x, outs, stream=stream)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            stage.forward(x, outs, stream=stream)
        b.record(stream)
        b.synchronize()
    ms = a.elapsed_time(b) / reps
    flops = sum(2.0 * m_ * n * k for _, m_, n, k in bev_layers())
    tflops = flops / (ms * 1e-3) / 1e12
    hw = BEV_HW * BEV_HW
    nbytes = 4 * hw * (336 + 512 + 128 + 10) + 2 * sum(n * k for _, _, n, k in bev_layers())
    out = {"workload": "BEV stage (fuser + SECOND backbone/deblocks + TransFusion shared conv "
                       "and heatmap head), 1 x 336 x 180 x 180 input, random-init weights "
                       "N(0,0.02), fp16 MFMA operands, fp32 accumulate",
           "ms": round(ms, 4), "tflops": round(tflops, 1), "gflop": round(flops / 1e9, 1),
           "reference_rtx4060ti_ms": BEV_REFERENCE["gpu_ms"],
           "resident_mib": round(stage.resident_bytes() / 2**20, 1),
           "roofline": {"kernel": "bev stage forward (18 convolutions)", "bound": "mfma",
                        "achieved": round(tflops, 1), "peak": PEAK_BF16_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                        "traffic": None, "algorithmic_bytes": nbytes,
                        "note": "dense fp16 MFMA peak equals the bf16 one (2.5 PFLOP/s)"}}
    stage.close()
    return out, path


def bev_cpu_baseline(path, seed=0):
    """The reference's CPU BEV stage (oracle/_ref, src/bev_stage.c, OpenMP) at
    a bounded 90x90 sample, scaled to 180x180 by the work ratio (4x)."""
    import oracle
    from bfhip import bfw
    kind = "reference" if oracle.available("ref_o3") else "port"
    o = oracle.Oracle("ref_o3" if kind == "reference" else "port")
    x = bfw.synthetic_bev(seed, BEV_HW // 2, BEV_HW // 2)
    with o.open_model(path) as m:
        t0 = time.perf_counter()
        o.bev_stage(m, x)
        t1 = time.perf_counter()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count()
    return {"value": round((t1 - t0) * 1e3 * 4, 1), "unit": "ms/forward", "cores": threads,
            "kind": kind, "backend": o.backend(),
            "sample": f"90x90 BEV ({1e3 * (t1 - t0):.0f} ms), scaled x4 to 180x180",
            "reference_readme_ms": BEV_REFERENCE["cpu_ms"], "cpu_model": _cpu_model()}


TF_HW, TF_PROPOSALS = 180, 200
# Reference TransFusion decoder on the RTX 4060 Ti, promoted 8-query tile
# flash attention, warm median of 5 processes (benchmark.csv:7).
TF_REFERENCE_MS = 17.164


def tf_flops(h=TF_HW, w=TF_HW, p=TF_PROPOSALS):
    """Algorithmic FLOPs of one decoder forward: key-side position head and
    K/V projections, cross attention (QK^T and PV), and the per-proposal
    dense layers and self attention."""
    keys, c = h * w, 128
    key_side = 2.0 * keys * c * (c + 2 * c)
    cross = 2.0 * 2 * p * keys * c
    rows = 2.0 * p * c * (c + 3 * c + c + c + c + 2 * c + 2 * c + 3 * c) + 2.0 * p * 20 * 64
    self_attn = 2.0 * 2 * p * p * c
    return key_side + cross + rows + self_attn, cross


def tf_leg(dev, reps, seed=0):
    """TransFusion decoder at 180x180 with 200 proposals: ms per forward
    (graph replay and eager), TFLOP/s against the MFMA roof."""
    import torch
    import bfhip
    from bfhip import bfw
    tmp = pathlib.Path(tempfile.mkdtemp(prefix="tf_"))
    path = bfw.write_transfusion(tmp / "tf.bfw", seed=seed, mode="baseline")
    sh, hm = (torch.from_numpy(a).to(dev) for a in bfw.synthetic_transfusion_inputs(seed, TF_HW, TF_HW))
    stream = torch.cuda.Stream()
    with bfhip.Model(path) as m:
        dec = bfhip.TransFusion(m, TF_HW, TF_HW, TF_PROPOSALS)
    with torch.cuda.stream(stream):
        outs = dec.forward(sh, hm, stream=stream)
        for _ in range(3):
            dec.forward(sh, hm, outs, stream=stream)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            dec.forward(sh, hm, outs, stream=stream)
        b.record(stream)
        b.synchronize()
        eager_ms = a.elapsed_time(b) / reps
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            dec.forward(sh, hm, outs, stream=stream)
        graph.replay()
        a.record(stream)
        for _ in range(reps):
            graph.replay()
        b.record(stream)
        b.synchronize()
        ms = a.elapsed_time(b) / reps
        dets = dec.decode(outs, 0.1, stream=stream)
    flops, cross = tf_flops()
    tflops = flops / (ms * 1e-3) / 1e12
    keys = TF_HW * TF_HW
    out = {"workload": "TransFusion decoder (NMS + top-200 proposals, self/cross attention, FFN, "
                       "six heads), 180 x 180 BEV map, random-init weights N(0,0.02); fp16 MFMA "
                       "operands on the key side and cross attention, fp32 elsewhere",
           "ms": round(ms, 4), "ms_eager": round(eager_ms, 4), "gflop": round(flops / 1e9, 2),
           "tflops": round(tflops, 1), "reference_rtx4060ti_ms": TF_REFERENCE_MS,
           "speedup_vs_reference": round(TF_REFERENCE_MS / ms, 1),
           "detections_at_0.1": dets.count,
           "resident_mib": round(dec.resident_bytes() / 2**20, 1),
           "roofline": {"kernel": "transfusion forward", "bound": "mfma",
                        "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                        "traffic": None,
                        "note": "dense fp16 MFMA peak; the cross attention's "
                                f"{8 * TF_PROPOSALS * keys / 1e6:.1f} M exponentials bound it "
                                "first (v_exp_f32 at a quarter of the VALU rate: ~5 us)"}}
    dec.close()
    return out, path


def tf_cpu_baseline(path, seed=0):
    """The reference's CPU TransFusion decoder (oracle/_ref: src/transfusion.c
    + src/transfusion_decoder.c, OpenMP) on the full 180x180 / 200-proposal
    workload."""
    import oracle
    from bfhip import bfw
    kind = "reference" if oracle.available("ref_o3") else "port"
    o = oracle.Oracle("ref_o3" if kind == "reference" else "port")
    sh, hm = bfw.synthetic_transfusion_inputs(seed, TF_HW, TF_HW)
    with o.open_model(path) as m:
        o.transfusion(m, sh, hm, TF_PROPOSALS)
        t0 = time.perf_counter()
        o.transfusion(m, sh, hm, TF_PROPOSALS)
        t1 = time.perf_counter()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count()
    return {"value": round((t1 - t0) * 1e3, 1), "unit": "ms/forward", "cores": threads,
            "kind": kind, "backend": o.backend(), "sample": "full 180x180 map, 200 proposals",
            "cpu_model": _cpu_model()}


LIDAR_POINTS, LIDAR_SWEEPS = 100000, 10  # the runtime frame's cloud: ~54k voxels
LIDAR_GRID = (41, 1440, 1440)
LIDAR_VOXELS, LIDAR_SPARSE = 160000, 160000  # the reference runtime's capacities
# Reference CUDA LiDAR branch, points -> LiDAR BEV, 100k points / 50k voxels,
# warm median (reference docs/draft.md:257-260).
LIDAR_REFERENCE_MS = 58.936


def _lidar_keys(s, dims):
    return (s[:, 0] * dims[1] + s[:, 1]) * dims[2] + s[:, 2]


def _subm_pairs(s, dims):
    import numpy as np
    keys = np.sort(_lidar_keys(s, dims))
    total = 0
    for dz in (-1, 0, 1):
        for dy in (-1, 0, 1):
            for dx in (-1, 0, 1):
                q = s + np.array([dz, dy, dx])
                ok = np.all((q >= 0) & (q < np.array(dims)), axis=1)
                k = _lidar_keys(q[ok], dims)
                pos = np.searchsorted(keys, k)
                pos[pos == len(keys)] = 0
                total += int((keys[pos] == k).sum())
    return total


def _strided(s, dims, kernel, stride, pad):
    """Output sites and (input, tap) pair count of a strided sparse conv."""
    import numpy as np
    out_dims = tuple((dims[a] + 2 * pad[a] - kernel[a]) // stride[a] + 1 for a in range(3))
    outs, pairs = [], 0
    for kz in range(kernel[0]):
        for ky in range(kernel[1]):
            for kx in range(kernel[2]):
                n = s + np.array(pad) - np.array([kz, ky, kx])
                ok = np.all((n >= 0) & (n % np.array(stride) == 0), axis=1)
                o = n[ok] // np.array(stride)
                ok2 = np.all(o < np.array(out_dims), axis=1)
                outs.append(o[ok2])
                pairs += int(ok2.sum())
    return np.unique(np.concatenate(outs), axis=0), out_dims, pairs


def lidar_work(coords, dims=LIDAR_GRID):
    """Algorithmic flops of the SECOND encoder on these voxel sites: 2 Ci Co
    per (output site, active tap) pair, per layer; and the site counts."""
    import numpy as np
    s = np.asarray(coords, np.int64)[:, 1:]
    flops, sites = 0, [len(s)]
    pairs = _subm_pairs(s, dims)
    flops += 2 * pairs * 5 * 16 + 4 * 2 * pairs * 16 * 16
    ch = (16, 32, 64, 128)
    for st in range(1, 4):
        s, dims, p = _strided(s, dims, (3, 3, 3), (2, 2, 2), (1 if st < 3 else 0, 1, 1))
        sites.append(len(s))
        flops += 2 * p * ch[st - 1] * ch[st] + 4 * 2 * _subm_pairs(s, dims) * ch[st] ** 2
    s, dims, p = _strided(s, dims, (3, 1, 1), (2, 1, 1), (0, 0, 0))
    sites.append(len(s))
    flops += 2 * p * 128 * 128
    return flops, sites


def lidar_leg(dev, reps, seed=0):
    """LiDAR branch on the reference's stress frame (100k points, two per voxel,
    50k voxels; bfw.stress_points): depth raster into the six camera images,
    voxeliser + MeanVFE, SECOND sparse encoder to the dense [256,180,180] BEV;
    ms per frame (eager and graph replay)."""
    import torch
    import bfhip
    from bfhip import bfw, frame_scene
    tmp = pathlib.Path(tempfile.mkdtemp(prefix="lidar_"))
    path = bfw.write_lidar_backbone(tmp / "lidar.bfw", seed=seed, mode="fan_in", gain=1.2)
    cal = frame_scene.calibration(seed)
    pts_np = bfw.stress_points(LIDAR_POINTS)
    t = lambda a: torch.from_numpy(a).to(dev)
    pts = t(pts_np)
    aug, l2i, post = t(cal["lidar_augmentation"]), t(cal["lidar_to_image"]), t(cal["image_augmentation"])
    stream = torch.cuda.Stream()
    raster = bfhip.DepthRaster(300000)
    vox = bfhip.Voxelizer(bfhip.voxel_config(LIDAR_VOXELS), 300000)
    with bfhip.Model(path) as m:
        net = bfhip.LidarBackbone(m, 1, *LIDAR_GRID, LIDAR_SPARSE)
    depth = torch.empty((6, 256, 704), device=dev)
    coords = torch.empty((LIDAR_VOXELS, 4), dtype=torch.int32, device=dev)
    means = torch.empty((LIDAR_VOXELS, 5), device=dev)
    count = torch.empty((1,), dtype=torch.int32, device=dev)
    bev = torch.empty(net.out_shape, device=dev)

    def frame():
        raster.forward(pts, aug, l2i, post, out=depth, stream=stream)
        vox.forward(pts, coords, means, count, stream=stream)
        net.forward(coords, means, count, out=bev, stream=stream)

    def timed(fn, n):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(n):
            fn()
        b.record(stream)
        b.synchronize()
        return a.elapsed_time(b) / n

    with torch.cuda.stream(stream):
        for _ in range(3):
            frame()
        eager_ms = timed(frame, reps)
        parts = {"depth_raster": timed(lambda: raster.forward(pts, aug, l2i, post, out=depth,
                                                              stream=stream), reps),
                 "voxelize": timed(lambda: vox.forward(pts, coords, means, count, stream=stream),
                                   reps),
                 "sparse_encoder": timed(lambda: net.forward(coords, means, count, out=bev,
                                                             stream=stream), reps)}
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            frame()
        graph.replay()
        ms = timed(graph.replay, reps)
    stream.synchronize()
    n = int(count.item())
    flops, sites = lidar_work(coords[:n].cpu().numpy())
    enc_ms = parts["sparse_encoder"]
    tflops = flops / (enc_ms * 1e-3) / 1e12
    out = {"workload": f"LiDAR branch, the reference's stress frame ({LIDAR_POINTS} points, two per "
                       f"voxel) -> depth raster (6 x 256 x 704) + voxeliser/MeanVFE ({n} voxels) "
                       "+ SECOND sparse encoder on the 41 x 1440 x 1440 grid -> [256,180,180] "
                       "BEV; random-init weights; split fp16 MFMA operands (hi + lo), fp32 "
                       "accumulation",
           "ms": round(ms, 4), "ms_eager": round(eager_ms, 4),
           "parts_ms": {k: round(v, 4) for k, v in parts.items()},
           "voxels": n, "sites_per_level": sites, "encoder_gflop": round(flops / 1e9, 2),
           "reference_rtx4060ti_ms": LIDAR_REFERENCE_MS,
           "speedup_vs_reference": round(LIDAR_REFERENCE_MS / ms, 1),
           "resident_mib": round((raster.resident_bytes() + vox.resident_bytes() +
                                  net.resident_bytes()) / 2**20, 1),
           "roofline": {"kernel": "sparse encoder forward", "bound": "mfma",
                        "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                        "traffic": None,
                        "note": "algorithmic flops (2 Ci Co per active (site, tap) pair) over "
                                "the encoder's time; the kernels issue three fp16 MFMAs per "
                                "product (split operands) and pad each wave's taps"}}
    for ctx in (raster, vox, net):
        ctx.close()
    return out, (path, pts_np)


def lidar_cpu_baseline(path, pts):
    """The reference's CPU LiDAR branch (oracle/_ref: src/voxel.c,
    src/kernels_ref.c MeanVFE, src/lidar_backbone.c) on the same frame."""
    import oracle
    kind = "reference" if oracle.available("ref_o3") else "port"
    o = oracle.Oracle("ref_o3" if kind == "reference" else "port")
    cfg = oracle.voxel_config(LIDAR_VOXELS)
    with o.open_model(path) as m:
        t0 = time.perf_counter()
        vx, c, cnt, _ = o.voxelize(pts, cfg)
        f = o.mean_vfe(vx, cnt)
        o.lidar_backbone(m, c, f, *LIDAR_GRID, capacity=LIDAR_SPARSE)
        t1 = time.perf_counter()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count()
    return {"value": round((t1 - t0) * 1e3, 1), "unit": "ms/frame", "cores": threads,
            "kind": kind, "backend": o.backend(),
            "sample": f"voxeliser + MeanVFE + sparse encoder on the full {LIDAR_POINTS}-point stress frame",
            "cpu_model": _cpu_model()}


# Reference CUDA runtime, real nuScenes mini frame, warm wall median
# (reference docs/draft.md:262-266).
RUNTIME_REFERENCE_MS = 142.381


def runtime_leg(reps, seed=1):
    """The full frame through bf_cuda_runtime_infer: host frame in (images,
    100k points, calibration), detections out; wall-clock ms per frame with
    the H2D copies, the graph replays and the D2H copy of the detections."""
    import bfhip
    from bfhip import bfw, frame_scene
    tmp = pathlib.Path(tempfile.mkdtemp(prefix="rt_"))
    path = bfw.write_full_model(tmp / "full.bfw", seed=seed)
    frame = frame_scene.frame(seed, LIDAR_POINTS, sweeps=LIDAR_SWEEPS)
    fi, keep = bfhip.frame_input(frame)
    with bfhip.Runtime(path, 300000, LIDAR_VOXELS, LIDAR_SPARSE) as rt:
        t0 = time.perf_counter()
        dets = rt.infer(fi)
        cold_ms = (time.perf_counter() - t0) * 1e3
        for _ in range(3):
            rt.infer(fi)
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            rt.infer(fi)
            times.append((time.perf_counter() - t0) * 1e3)
        resident = rt.resident_bytes()
    times.sort()
    ms = times[len(times) // 2]
    h2d = sum(keep[k].nbytes for k in keep)
    del keep
    return {"workload": f"full frame: 6 x 3 x 256 x 704 images + {LIDAR_POINTS} points "
                        f"({LIDAR_SWEEPS} sweeps) -> detections; random-init checkpoint "
                        "(N(0, 1/fan_in) weights); LiDAR and camera branches concurrent in HIP graphs",
            "ms": round(ms, 3), "ms_min": round(times[0], 3), "cold_ms": round(cold_ms, 1),
            "detections": dets.count, "h2d_mib": round(h2d / 2**20, 1),
            "resident_mib": round(resident / 2**20, 1),
            "reference_rtx4060ti_ms": RUNTIME_REFERENCE_MS,
            "speedup_vs_reference": round(RUNTIME_REFERENCE_MS / ms, 1)}, (path, frame)


def runtime_cpu_baseline(path, frame):
    """The reference's CPU frame runtime (oracle/_ref: src/runtime.c and its
    modules, OpenMP) on the same frame."""
    import oracle
    kind = "reference" if oracle.available("ref_o3") else "port"
    o = oracle.Oracle("ref_o3" if kind == "reference" else "port")
    t0 = time.perf_counter()
    o.runtime_infer(path, frame, 300000, LIDAR_VOXELS, LIDAR_SPARSE)
    t1 = time.perf_counter()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count()
    return {"value": round((t1 - t0) * 1e3, 1), "unit": "ms/frame", "cores": threads,
            "kind": kind, "backend": o.backend(), "sample": "the same full frame, once",
            "cpu_model": _cpu_model()}


def cpu_baseline(model_path, cameras):
    """Reference CPU path (oracle/_ref/libbfref_o3.so: the reference's C
    compiled from its own sources under its own -O3 OpenMP CFLAGS) on
    `cameras` cameras, scaled to a 6-camera frame when fewer.  Falls back to
    the restatement if the reference build is absent."""
    import oracle
    from bfhip import bfw
    flavour = "ref_o3" if oracle.available("ref_o3") else "port"
    o = oracle.Oracle(flavour)
    images = bfw.synthetic_images(0, cameras, 256, 704)
    depth = bfw.synthetic_depth(0, cameras, 256, 704)
    with o.open_model(model_path) as m:
        t0 = time.perf_counter()
        s0, s1, s2 = o.swin_backbone(m, images)
        t1 = time.perf_counter()
        f0, _ = o.image_fpn(m, s0, s1, s2)
        o.depth_head(m, f0, depth)
        t2 = time.perf_counter()
    per_frame_ms = (t2 - t0) * 1e3 * 6 / cameras
    sample = (f"{cameras} of 6 cameras" if cameras < 6 else "one full 6-camera frame") + \
        f", Swin-T + FPN + depth head at 256x704 (swin {1e3 * (t1 - t0):.0f} ms, " \
        f"neck {1e3 * (t2 - t1):.0f} ms)" + (f", scaled x{6 / cameras:g}" if cameras < 6 else "")
    out = {"value": round(per_frame_ms, 1), "unit": "ms/frame",
           "kind": "reference" if flavour == "ref_o3" else "port", "backend": o.backend(),
           "build": "-O3 -std=c11 -fopenmp -DBF_WITH_OPENMP (reference Makefile:4,40-45)"
                    if flavour == "ref_o3" else "restatement", "sample": sample}
    out.update(_cpu_host())
    return out


def _cpu_host():
    """Host facts for a CPU figure: the threads OpenMP used (`cores`), nproc,
    the process's CPU affinity and the CPU model."""
    aff = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else []
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or len(aff) or os.cpu_count()
    return {"cores": threads, "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "nproc": os.cpu_count(), "affinity_cpus": len(aff),
            "affinity": _ranges(aff), "cpu_model": _cpu_model()}


def _ranges(cpus):
    out, i = [], 0
    while i < len(cpus):
        j = i
        while j + 1 < len(cpus) and cpus[j + 1] == cpus[j] + 1:
            j += 1
        out.append(f"{cpus[i]}-{cpus[j]}" if j > i else f"{cpus[i]}")
        i = j + 1
    return ",".join(out)


def _cpu_model():
    import subprocess
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in txt.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    args = parse()
    if args.pmc_child:
        pmc_child(args.pmc_child)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the path shards per camera "
                                   "across GPUs by design (DESIGN.md) but no multi-GPU run is "
                                   "part of it", "n_gpus": args.gpus}))
        sys.exit(2)
    import numpy as np
    import torch
    import bfhip
    from bfhip import bfw

    dev = torch.device("cuda:0")
    tmp = pathlib.Path(tempfile.mkdtemp(prefix="bench_"))
    model_path = bfw.write_camera_branch(tmp / "camera_branch.bfw", seed=0, mode="baseline")
    with bfhip.Model(model_path) as m:
        swin = bfhip.Swin(m, 6, 256, 704)
        neck = bfhip.CameraNeck(m, 6, 32, 88, DOWN_IN_HW, DOWN_IN_HW)

    frames = 20
    imgs = [torch.from_numpy(bfw.synthetic_images(s, 6, 256, 704)).to(dev) for s in range(frames)]
    deps = [torch.from_numpy(bfw.synthetic_depth(s, 6, 256, 704)).to(dev) for s in range(frames)]
    outs = [torch.empty(s, device=dev) for s in swin.output_shapes()]
    logits = torch.empty((6, 118, 32, 88), device=dev)
    ctx = torch.empty((6, 80, 32, 88), device=dev)

    # Every frame's inputs stay resident; step i reads frame i % frames in
    # place, as the reference's forward reads its device input (no staging
    # copy inside the timed region).
    def step(i):
        swin.forward(imgs[i], outs)
        neck.neck_forward(*outs, deps[i], logits, ctx)

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        step(0)
        torch.cuda.synchronize()
        eager = (logits.clone(), ctx.clone())
        runs = [functools.partial(step, i) for i in range(frames)]
        if not args.no_graph:
            # One captured graph per resident frame (the kernel arguments
            # differ only in the input pointers); replay 0 must equal the
            # eager pass bit for bit.
            graphs = []
            for i in range(frames):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=stream):
                    step(i)
                graphs.append(g)
            graphs[0].replay()
            torch.cuda.synchronize()
            if not (torch.equal(eager[0], logits) and torch.equal(eager[1], ctx)):
                raise SystemExit("graph replay differs from eager forward")
            runs = [g.replay for g in graphs]

        for i in range(args.warmup):
            runs[i % frames]()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            runs[i % frames]()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    gflop = frame_flops() / 1e9
    gflop_exec = frame_flops(window_rows=False) / 1e9
    tflops = gflop / ms

    result = {
        "metric": "GEMM TFLOP/s (% bf16 MFMA peak); 6-cam Swin-T+FPN+depth ms/frame",
        "value": round(ms, 4),
        "unit": "ms/frame",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",  # fp16 MFMA operands, fp32 accumulation (dense fp16 peak = bf16 peak)
        "data": "synthetic (images U[0,1] ImageNet-normalised, dense depth |N(0,1)|, "
                "random-init weights N(0,0.02), seeds 0-19)",
        "config": {"workload": "BASELINE config 5: 6x3x256x704 images -> Swin-T -> FPN -> "
                               "depth head (118 bins + 80 ctx), one frame per step",
                   "cameras": 6, "image_hw": [256, 704], "graph": not args.no_graph,
                   "resident_frames": frames},
        "tflops": round(tflops, 2),
        "gflop_per_frame": round(gflop, 1),
        "gflop_note": "reference-equivalent work: QKV and proj charged at windows x 49 rows "
                      "(padding tokens included), as the reference computes them",
        "frac_bf16_peak": round(tflops / PEAK_BF16_TFLOPS, 4),
        "gflop_per_frame_executed": round(gflop_exec, 1),
        "tflops_executed": round(gflop_exec / ms, 2),
        "frac_bf16_peak_executed": round(gflop_exec / ms / PEAK_BF16_TFLOPS, 4),
        "frames_per_s": round(1e3 / ms, 1),
    }
    kernels = []
    if not args.no_roofline:
        io = neck_io(dev)
        with torch.cuda.stream(stream):
            only = tuple(k for k in args.kernels.split(",") if k)
            kernels = time_kernels(swin, neck, stream, io, args.kernel_reps, only)
        if not args.no_traffic:
            torch.cuda.synchronize()
            # The counter child launches the ops in op_table order.
            with torch.cuda.stream(stream):
                order = list(op_table(swin, neck, stream, io))
            counters, errors = measure_op_counters(order)
            for e in kernels:
                c = counters.get(e["kernel"], {})
                avg_s = e["avg_us"] / 1e6
                if "mfma_util_pct" in c:
                    e["mfma_util_pct"] = c["mfma_util_pct"]
                    e["mfma_flops_per_launch"] = c["mfma_flops"]
                    e["mfma_tflops"] = round(c["mfma_flops"] / avg_s / 1e12, 1)
                if "fetch_bytes" in c and "write_bytes" in c:
                    e["traffic"] = c["fetch_bytes"] + c["write_bytes"]
                    e["traffic_detail"] = {k: c[k] for k in ("fetch_bytes", "write_bytes",
                                                             "fetch_scale", "write_scale")}
                    e["traffic_gbs"] = round(e["traffic"] / avg_s / 1e9, 1)
            if errors:
                result["counter_errors"] = errors
        frame_ops = [e for e in kernels if not e["kernel"].startswith("neck.downsample")]
        if frame_ops:
            result["roofline"] = dict(frame_ops[0])
        keep = ("kernel", "bound", "frac", "avg_us", "us_per_frame", "tflops", "gbs",
                "mfma_util_pct", "mfma_tflops", "traffic", "traffic_gbs")
        result["kernels"] = [{k: e[k] for k in keep if k in e} for e in frame_ops]
    if not args.no_downsample:
        result["downsample"] = downsample_leg(neck, dev, stream, max(args.steps, 20),
                                              [{k: e[k] for k in ("kernel", "frac", "avg_us",
                                                                  "tflops", "mfma_util_pct")
                                                if k in e} for e in kernels])
    if not args.no_config1:
        result["config1"] = config1_leg(dev, 50, not args.no_cpu)
    if not args.no_calibrate:
        result["calibration"] = calibrate_leg(dev)
    if not args.no_library:
        result["library_gemm"] = library_gemm_leg(dev, kernels)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(model_path, args.cpu_cameras)
    if not args.no_lss:
        lss, sc = lss_leg(dev, max(args.steps, 20), not (args.no_roofline or args.no_traffic))
        if not args.no_cpu:
            lss["cpu_baseline"] = lss_cpu_baseline(sc)
        result["lss"] = lss
    if not args.no_bev:
        bev, bev_path = bev_leg(dev, max(args.steps, 20))
        if not args.no_cpu:
            bev["cpu_baseline"] = bev_cpu_baseline(bev_path)
        result["bev_stage"] = bev
    if not args.no_tf:
        tf, tf_path = tf_leg(dev, max(args.steps, 20))
        if not args.no_cpu:
            tf["cpu_baseline"] = tf_cpu_baseline(tf_path)
        result["transfusion"] = tf
    if not args.no_lidar:
        lidar, (lidar_path, lidar_pts) = lidar_leg(dev, max(args.steps, 20))
        if not args.no_cpu:
            lidar["cpu_baseline"] = lidar_cpu_baseline(lidar_path, lidar_pts)
        result["lidar"] = lidar
    if not args.no_runtime:
        rt, (rt_path, rt_frame) = runtime_leg(max(args.steps, 10))
        if not args.no_cpu:
            rt["cpu_baseline"] = runtime_cpu_baseline(rt_path, rt_frame)
        result["runtime"] = rt
    print(json.dumps(result))


if __name__ == "__main__":
    main()
