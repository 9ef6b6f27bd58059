"""Parity of the camera-neck context (bf_cuda_camera_*) against the CPU oracle.

Compact shapes are the reference's own (tests/test_cuda_camera.cu:54,78 and
the stage tests): FPN at 4x6, depth head at 2x3, downsample at 8x10.
Production shapes: FPN + depth head at 32x88 features (256x704 dense depth)
and the downsample on a 360x360 BEV.
"""

import numpy as np
import pytest

from util import assert_close

pytestmark = pytest.mark.gpu


def _rand(seed, shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def _swin_like(b, h, w, seed=0):
    h1, w1 = (h + 1) // 2, (w + 1) // 2
    h2, w2 = (h1 + 1) // 2, (w1 + 1) // 2
    return (_rand(seed, (b, 192, h, w)), _rand(seed + 1, (b, 384, h1, w1)),
            _rand(seed + 2, (b, 768, h2, w2)))


def _t(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def _neck(model_path, b, h, w, bev=(8, 10)):
    import bfhip
    with bfhip.Model(model_path) as m:
        return bfhip.CameraNeck(m, b, h, w, bev[0], bev[1])


@pytest.mark.parametrize("b,h,w", [(1, 4, 6), (2, 5, 7), (1, 32, 88)])
def test_fpn_matches_oracle(device, tmp_models, b, h, w):
    import oracle
    import torch
    path = tmp_models("fan_in", 1)
    s0, s1, s2 = _swin_like(b, h, w)
    neck = _neck(path, b, h, w)
    f0, f1 = neck.fpn_forward(_t(s0, device), _t(s1, device), _t(s2, device))
    torch.cuda.synchronize()
    o = oracle.Oracle("port")
    with o.open_model(path) as m:
        r0, r1 = o.image_fpn(m, s0, s1, s2)
    assert_close(f1.cpu().numpy(), r1, "fpn1")
    assert_close(f0.cpu().numpy(), r0, "fpn0")


@pytest.mark.parametrize("b,h,w", [(1, 2, 3), (2, 3, 5), (1, 32, 88)])
def test_depth_head_matches_oracle(device, tmp_models, b, h, w):
    import oracle
    import torch
    from bfhip import bfw
    path = tmp_models("fan_in", 1)
    feats = np.abs(_rand(5, (b, 256, h, w)))
    depth = bfw.synthetic_depth(2, b, 8 * h, 8 * w)
    neck = _neck(path, b, h, w)
    lg, cx = neck.depth_forward(_t(feats, device), _t(depth, device))
    torch.cuda.synchronize()
    o = oracle.Oracle("port")
    with o.open_model(path) as m:
        rl, rc = o.depth_head(m, feats, depth)
    assert_close(lg.cpu().numpy(), rl, "depth logits")
    assert_close(cx.cpu().numpy(), rc, "context")


@pytest.mark.parametrize("bev", [(8, 10), (360, 360), (12, 6)])
def test_downsample_matches_oracle(device, tmp_models, bev):
    import oracle
    import torch
    path = tmp_models("fan_in", 1)
    x = _rand(9, (1, 80, bev[0], bev[1]))
    neck = _neck(path, 1, 2, 3, bev)
    got = neck.downsample_forward(_t(x, device))
    torch.cuda.synchronize()
    o = oracle.Oracle("port")
    with o.open_model(path) as m:
        ref = o.lss_downsample(m, x)
    assert got.shape == ref.shape
    assert_close(got.cpu().numpy(), ref, f"downsample {bev}")


def test_neck_forward_equals_fpn_then_depth(device, tmp_models):
    """Production scheduling (context-owned FPN levels) is bit-identical to
    the two standalone boundaries, and matches the oracle chain."""
    import oracle
    import torch
    from bfhip import bfw
    path = tmp_models("fan_in", 1)
    b, h, w = 2, 32, 88
    s = _swin_like(b, h, w, seed=20)
    depth = bfw.synthetic_depth(4, b, 8 * h, 8 * w)
    neck = _neck(path, b, h, w)
    st = [_t(a, device) for a in s]
    dt = _t(depth, device)
    lg, cx = neck.neck_forward(*st, dt)
    f0, _ = neck.fpn_forward(*st)
    lg2, cx2 = neck.depth_forward(f0, dt)
    torch.cuda.synchronize()
    assert torch.equal(lg, lg2) and torch.equal(cx, cx2)
    o = oracle.Oracle("port")
    with o.open_model(path) as m:
        r0, _ = o.image_fpn(m, *s)
        rl, rc = o.depth_head(m, r0, depth)
    assert_close(lg.cpu().numpy(), rl, "neck logits")
    assert_close(cx.cpu().numpy(), rc, "neck context")


def test_neck_production_batch_invariance_and_repeat(device, tmp_models):
    """6x32x88 production neck (BASELINE config 4's camera shape; reference
    gate tests/test_cuda_camera_full.cu:69-72 repeats the production chain and
    compares bit for bit): repeated forwards are bit-identical, camera k of
    the 6-camera forward is bit-identical to the 1-camera forward of the same
    inputs (FPN levels, depth logits and context: no cross-camera coupling),
    and the last camera matches the oracle."""
    import oracle
    import torch
    from bfhip import bfw
    path = tmp_models("fan_in", 1)
    b, h, w = 6, 32, 88
    s = _swin_like(b, h, w, seed=31)
    depth = bfw.synthetic_depth(6, b, 8 * h, 8 * w)
    six = _neck(path, b, h, w, (360, 360))
    one = _neck(path, 1, h, w, (360, 360))
    st = [_t(a, device) for a in s]
    dt = _t(depth, device)
    lg, cx = six.neck_forward(*st, dt)
    lg2, cx2 = six.neck_forward(*st, dt)
    f0, f1 = six.fpn_forward(*st)
    torch.cuda.synchronize()
    assert torch.equal(lg, lg2) and torch.equal(cx, cx2), "repeat neck forward differs"
    for cam in (0, 3, 5):
        sl = [a[cam:cam + 1].contiguous() for a in st]
        lg1, cx1 = one.neck_forward(*sl, dt[cam:cam + 1].contiguous())
        g0, g1 = one.fpn_forward(*sl)
        torch.cuda.synchronize()
        assert torch.equal(lg[cam:cam + 1], lg1), f"camera {cam} logits depend on batch"
        assert torch.equal(cx[cam:cam + 1], cx1), f"camera {cam} context depends on batch"
        assert torch.equal(f0[cam:cam + 1], g0) and torch.equal(f1[cam:cam + 1], g1), \
            f"camera {cam} FPN levels depend on batch"
    o = oracle.Oracle("port")
    with o.open_model(path) as m:
        r0, _ = o.image_fpn(m, *[a[5:6] for a in s])
        rl, rc = o.depth_head(m, r0, depth[5:6])
    assert_close(lg[5:6].cpu().numpy(), rl, "camera 5 logits")
    assert_close(cx[5:6].cpu().numpy(), rc, "camera 5 context")
