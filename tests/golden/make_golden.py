#!/usr/bin/env python3
"""Write tests/golden/reference_vectors.npz from the reference's own C.

The reference's CPU sources are compiled from /root/reference into
oracle/_ref (oracle/Makefile, `make ref`); this script runs that library on
the scalar path (BF_CPU_SCALAR=1, no OpenMP) over small deterministic inputs
at the reference's test shapes and stores inputs and outputs.  The vectors
pin the oracle restatement wherever the reference itself is absent (the GPU
box, later sessions).  Module vectors use the synthetic fan-in checkpoint,
which bfhip/bfw.py regenerates bit-identically from its seed.

Usage: python tests/golden/make_golden.py   (needs oracle/_ref built)
"""

import pathlib
import sys
import tempfile

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "bevfusion.c_amd"), str(ROOT / "tests")]

import oracle  # noqa: E402
from bfhip import bfw  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent / "reference_vectors.npz"


def main():
    ref = oracle.Oracle("ref_scalar")
    r = np.random.default_rng(20260718)
    v = {}
    # kernels (test_kernels.c shapes)
    v["conv.x"] = r.standard_normal((2, 4, 5, 6)).astype(np.float32)
    v["conv.w"] = r.standard_normal((6, 2, 3, 3)).astype(np.float32)
    v["conv.b"] = r.standard_normal(6).astype(np.float32)
    v["linear.x"] = r.standard_normal((7, 5)).astype(np.float32)
    v["linear.w"] = r.standard_normal((4, 5)).astype(np.float32)
    v["linear.b"] = r.standard_normal(4).astype(np.float32)
    v["ln.x"] = r.standard_normal((5, 7)).astype(np.float32)
    v["ln.g"] = r.standard_normal(7).astype(np.float32)
    v["ln.b"] = r.standard_normal(7).astype(np.float32)
    v["softmax.x"] = (r.standard_normal((4, 9)) * 4).astype(np.float32)
    v["softmax.x"][0, 0], v["softmax.x"][1, 1] = 100.0, -100.0
    v["gelu.x"] = np.linspace(-8, 8, 65).astype(np.float32)
    # window attention (test_swin.c shape: B2 5x7 C8 heads 2 window 3)
    c, heads, window = 8, 2, 3
    v["swin.query"] = r.standard_normal((2, 5, 7, c)).astype(np.float32)
    v["swin.qkv_w"] = (r.standard_normal((3 * c, c)) * 0.25).astype(np.float32)
    v["swin.qkv_b"] = (r.standard_normal(3 * c) * 0.1).astype(np.float32)
    v["swin.rel_bias"] = (r.standard_normal((25, heads)) * 0.05).astype(np.float32)
    v["swin.rel_index"] = bfw.relative_position_index(window)
    v["swin.proj_w"] = (r.standard_normal((c, c)) * 0.25).astype(np.float32)
    v["swin.proj_b"] = (r.standard_normal(c) * 0.1).astype(np.float32)
    # module inputs (compact stage-test shapes)
    v["images"] = bfw.synthetic_images(3, 1, 32, 48)
    v["fpn.s0"] = r.standard_normal((1, 192, 4, 6)).astype(np.float32)
    v["fpn.s1"] = r.standard_normal((1, 384, 2, 3)).astype(np.float32)
    v["fpn.s2"] = r.standard_normal((1, 768, 1, 2)).astype(np.float32)
    v["depth.features"] = np.abs(r.standard_normal((1, 256, 2, 3))).astype(np.float32)
    v["depth.dense"] = bfw.synthetic_depth(3, 1, 16, 24)
    v["down.bev"] = r.standard_normal((1, 80, 8, 10)).astype(np.float32)

    with oracle.scalar_env():
        v["conv.out"] = ref.conv2d(v["conv.x"], v["conv.w"], v["conv.b"], (2, 2), (1, 1), groups=2)
        v["linear.out"] = ref.linear(v["linear.x"], v["linear.w"], v["linear.b"])
        v["ln.out"] = ref.layer_norm(v["ln.x"], v["ln.g"], v["ln.b"])
        v["softmax.out"] = ref.softmax(v["softmax.x"])
        v["gelu.out"] = ref.gelu(v["gelu.x"])
        args = {k.split(".", 1)[1]: v[k] for k in v if k.startswith("swin.")}
        for shift in (0, 1):
            v[f"swin.out_shift{shift}"] = ref.swin_window(heads=heads, window=window, shift=shift, **args)
        with tempfile.TemporaryDirectory() as tmp:
            path = bfw.write_camera_branch(pathlib.Path(tmp) / "m.bfw", seed=1, mode="fan_in")
            with ref.open_model(path) as m:
                for i, o in enumerate(ref.swin_backbone(m, v["images"])):
                    v[f"swin_backbone.out{i}"] = o
                v["fpn.out0"], v["fpn.out1"] = ref.image_fpn(m, v["fpn.s0"], v["fpn.s1"], v["fpn.s2"])
                v["depth.logits"], v["depth.context"] = ref.depth_head(m, v["depth.features"],
                                                                       v["depth.dense"])
                v["down.out"] = ref.lss_downsample(m, v["down.bev"])
    np.savez_compressed(OUT, **v)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(v)} arrays)")


if __name__ == "__main__":
    main()
