"""The oracle restatement against the reference's own C, compiled from its
sources into oracle/_ref (CPU only; skipped where the reference is absent).

Scalar builds with BF_CPU_SCALAR=1 must agree bit for bit: same operation
order per element.  OpenMP builds use `omp simd` reductions whose order the
compiler picks, so they are held to 1e-6 relative instead.
"""

import numpy as np
import pytest

import oracle
from bfhip import bfw

pytestmark = pytest.mark.skipif(not oracle.available("ref_scalar"),
                                reason="oracle/_ref not built (no /root/reference)")


@pytest.fixture(scope="module")
def libs():
    return oracle.Oracle("port_scalar"), oracle.Oracle("ref_scalar")


@pytest.fixture(scope="module")
def omp_libs():
    return oracle.Oracle("port"), oracle.Oracle("ref")


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    return bfw.write_camera_branch(tmp_path_factory.mktemp("m") / "m.bfw", seed=1, mode="fan_in")


def same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def rng(s):
    return np.random.default_rng(s)


def test_backends(libs, omp_libs):
    with oracle.scalar_env():
        assert libs[0].backend() == libs[1].backend() == "scalar-forced"
    assert omp_libs[0].backend() == omp_libs[1].backend() == "openmp"


@pytest.mark.parametrize("case", [
    ((2, 4, 5, 6), (6, 2, 3, 3), (2, 2), (1, 1), 2),
    ((1, 8, 33, 29), (16, 8, 5, 5), (4, 4), (2, 2), 1),
    ((1, 64, 5, 7), (11, 64, 1, 1), (1, 1), (0, 0), 1),
    ((2, 3, 9, 10), (5, 3, 3, 3), (2, 1), (1, 0), 1),
])
def test_conv_bit_exact(libs, case):
    xs, ws, stride, pad, groups = case
    x = rng(1).standard_normal(xs).astype(np.float32)
    w = rng(2).standard_normal(ws).astype(np.float32)
    b = rng(3).standard_normal(ws[0]).astype(np.float32)
    with oracle.scalar_env():
        a = libs[0].conv2d(x, w, b, stride, pad, groups=groups)
        r = libs[1].conv2d(x, w, b, stride, pad, groups=groups)
    assert same(a, r)
    # The sweep path (dispatch without BF_CPU_SCALAR) also matches bitwise.
    assert same(libs[0].conv2d(x, w, b, stride, pad, groups=groups),
                libs[1].conv2d(x, w, b, stride, pad, groups=groups))


def test_conv_transpose_bit_exact(libs):
    x = rng(4).standard_normal((2, 4, 5, 6)).astype(np.float32)
    w = rng(5).standard_normal((4, 3, 2, 2)).astype(np.float32)
    b = rng(6).standard_normal(3).astype(np.float32)
    assert same(libs[0].conv_transpose2d(x, w, b, stride=(2, 2)),
                libs[1].conv_transpose2d(x, w, b, stride=(2, 2)))


def test_pointwise_bit_exact(libs):
    x = (rng(7).standard_normal((31, 64)) * 2).astype(np.float32)
    w = rng(8).standard_normal((48, 64)).astype(np.float32)
    b = rng(9).standard_normal(48).astype(np.float32)
    g, bb = rng(10).standard_normal(64).astype(np.float32), rng(11).standard_normal(64).astype(np.float32)
    s = (rng(12).standard_normal((4, 9)) * 4).astype(np.float32)
    s[0, 0], s[1, 1] = 100, -100
    v = np.linspace(-8, 8, 65).astype(np.float32)
    bn = [rng(13 + i).standard_normal(3).astype(np.float32) for i in range(3)]
    var = (rng(16).random(3) + 0.2).astype(np.float32)
    t = rng(17).standard_normal((2, 3, 4, 5)).astype(np.float32)
    with oracle.scalar_env():
        p, r = libs
        assert same(p.linear(x, w, b), r.linear(x, w, b))
        assert same(p.layer_norm(x, g, bb), r.layer_norm(x, g, bb))
        assert same(p.softmax(s), r.softmax(s))
        assert same(p.gelu(v), r.gelu(v))
        assert same(p.relu(v), r.relu(v))
        assert same(p.batch_norm(t, *bn, var, eps=1e-3), r.batch_norm(t, *bn, var, eps=1e-3))


@pytest.mark.parametrize("shape", [(2, 5, 7, 8, 2, 3, 0), (2, 5, 7, 8, 2, 3, 1),
                                   (1, 9, 11, 32, 1, 7, 3), (1, 8, 22, 64, 2, 7, 3)])
@pytest.mark.parametrize("streamed", [True, False])
def test_window_attention_bit_exact(libs, shape, streamed):
    import torchref
    b, h, w, c, heads, window, shift = shape
    r = rng(sum(shape))
    case = dict(
        query=r.standard_normal((b, h, w, c)).astype(np.float32),
        qkv_w=(r.standard_normal((3 * c, c)) * 0.25).astype(np.float32),
        qkv_b=(r.standard_normal(3 * c) * 0.1).astype(np.float32),
        rel_bias=(r.standard_normal(((2 * window - 1) ** 2, heads)) * 0.05).astype(np.float32),
        rel_index=torchref.relative_position_index(window).numpy().astype(np.int64),
        proj_w=(r.standard_normal((c, c)) * 0.25).astype(np.float32),
        proj_b=(r.standard_normal(c) * 0.1).astype(np.float32))
    with oracle.scalar_env():
        a = libs[0].swin_window(heads=heads, window=window, shift=shift, streamed=streamed, **case)
        e = libs[1].swin_window(heads=heads, window=window, shift=shift, streamed=streamed, **case)
    assert same(a, e)


def _modules(o, path, seed=3):
    images = bfw.synthetic_images(seed, 1, 32, 48)
    r = rng(seed)
    s0 = r.standard_normal((1, 192, 4, 6)).astype(np.float32)
    s1 = r.standard_normal((1, 384, 2, 3)).astype(np.float32)
    s2 = r.standard_normal((1, 768, 1, 2)).astype(np.float32)
    feats = np.abs(r.standard_normal((1, 256, 2, 3))).astype(np.float32)
    depth = bfw.synthetic_depth(seed, 1, 16, 24)
    bev = r.standard_normal((1, 80, 8, 10)).astype(np.float32)
    with o.open_model(path) as m:
        return (*o.swin_backbone(m, images), *o.image_fpn(m, s0, s1, s2),
                *o.depth_head(m, feats, depth), o.lss_downsample(m, bev))


def test_modules_bit_exact(libs, model):
    """The reference's compact stage-test shapes: Swin 32x48 (test_swin_backbone.c),
    FPN 4x6 (test_image_fpn.c), depth 2x3 (test_depth_head.c), downsample 8x10
    (test_lss_downsample.c)."""
    with oracle.scalar_env():
        a = _modules(libs[0], model)
        r = _modules(libs[1], model)
    for x, y in zip(a, r):
        assert x.shape == y.shape and same(x, y)


def test_modules_openmp_close(omp_libs, model):
    a = _modules(omp_libs[0], model)
    r = _modules(omp_libs[1], model)
    for x, y in zip(a, r):
        assert np.max(np.abs(x - y)) <= 1e-6 * max(1.0, np.max(np.abs(y)))


def test_workspace_sizes_and_rejection(libs):
    import ctypes as C
    p, r = (l.lib for l in libs)
    for fn, args in (("bf_swin_backbone_workspace_bytes", (6, 256, 704)),
                     ("bf_image_fpn_workspace_bytes", (32, 88)),
                     ("bf_depth_head_workspace_bytes", (32, 88)),
                     ("bf_lss_downsample_workspace_bytes", (360, 360))):
        assert getattr(p, fn)(*args) == getattr(r, fn)(*args) > 0
    assert p.bf_lss_downsample_workspace_bytes(361, 360) == r.bf_lss_downsample_workspace_bytes(361, 360) == 0
    d = oracle.WindowDesc(1, 7, 7, 96, 3, 7, 3)
    assert p.bf_swin_shifted_window_workspace_bytes(C.byref(d)) == \
        r.bf_swin_shifted_window_workspace_bytes(C.byref(d))


def test_workspace_minus_one_rejected(model):
    """Both implementations reject workspace_bytes - 1 (test_swin_backbone.c:54-77)."""
    import ctypes as C
    for fl in ("port_scalar", "ref_scalar"):
        o = oracle.Oracle(fl)
        with o.open_model(model) as m:
            net = m.create("lss_downsample")
            need = o.lib.bf_lss_downsample_workspace_bytes(8, 10)
            x = np.zeros((1, 80, 8, 10), np.float32)
            out = np.zeros((1, 80, 5, 4), np.float32)
            ws = np.zeros(need // 4 + 1, np.float32)
            err = C.create_string_buffer(128)
            assert not o.lib.bf_lss_downsample_forward_ref(net, x, 1, 8, 10, out, ws.ctypes.data,
                                                           need - 1, err, 128)
            assert o.lib.bf_lss_downsample_forward_ref(net, x, 1, 8, 10, out, ws.ctypes.data,
                                                       need, err, 128)
            o.lib.bf_lss_downsample_destroy(net)
