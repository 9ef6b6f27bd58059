"""The oracle restatement reproduces the reference's golden vectors bit for
bit (tests/golden/reference_vectors.npz, written from the reference's own C by
tests/golden/make_golden.py).  CPU only; runs without /root/reference."""

import pathlib
import tempfile

import numpy as np
import pytest

import oracle
from bfhip import bfw

GOLD = pathlib.Path(__file__).resolve().parent / "golden" / "reference_vectors.npz"


@pytest.fixture(scope="module")
def g():
    with np.load(GOLD, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.fixture(scope="module")
def port():
    return oracle.Oracle("port_scalar")


def same(a, b):
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_kernel_vectors(g, port):
    with oracle.scalar_env():
        assert same(port.conv2d(g["conv.x"], g["conv.w"], g["conv.b"], (2, 2), (1, 1), groups=2),
                    g["conv.out"])
        assert same(port.linear(g["linear.x"], g["linear.w"], g["linear.b"]), g["linear.out"])
        assert same(port.layer_norm(g["ln.x"], g["ln.g"], g["ln.b"]), g["ln.out"])
        assert same(port.softmax(g["softmax.x"]), g["softmax.out"])
        assert same(port.gelu(g["gelu.x"]), g["gelu.out"])


@pytest.mark.parametrize("shift", [0, 1])
def test_window_attention_vectors(g, port, shift):
    args = {k.split(".", 1)[1]: g[k] for k in g if k.startswith("swin.") and "out" not in k}
    with oracle.scalar_env():
        got = port.swin_window(heads=2, window=3, shift=shift, **args)
    assert same(got, g[f"swin.out_shift{shift}"])


def test_module_vectors(g, port):
    with tempfile.TemporaryDirectory() as tmp:
        path = bfw.write_camera_branch(pathlib.Path(tmp) / "m.bfw", seed=1, mode="fan_in")
        with oracle.scalar_env(), port.open_model(path) as m:
            for i, o in enumerate(port.swin_backbone(m, g["images"])):
                assert same(o, g[f"swin_backbone.out{i}"]), f"swin output {i}"
            f0, f1 = port.image_fpn(m, g["fpn.s0"], g["fpn.s1"], g["fpn.s2"])
            assert same(f0, g["fpn.out0"]) and same(f1, g["fpn.out1"])
            lg, cx = port.depth_head(m, g["depth.features"], g["depth.dense"])
            assert same(lg, g["depth.logits"]) and same(cx, g["depth.context"])
            assert same(port.lss_downsample(m, g["down.bev"]), g["down.out"])
