"""CPU checks of the BEV-stage oracle (oracle/src/bev_stage.c).

Pinned by (a) the reference's own src/bev_stage.c compiled as-is
(oracle/_ref): bit-identical on the scalar path at the reference test's 8x8
shape (tests/test_bev_stage.c:53) and a non-square one; (b) an independent
float64 PyTorch restatement (F.conv2d / F.conv_transpose2d / F.batch_norm with
epsilon 1e-3, torch.cat), so a wrong layer order, stride, transposed-weight
layout or BN epsilon fails; (c) the reference test's workspace - 1 and
odd-size rejections (tests/test_bev_stage.c:66-68).
"""

import ctypes as C

import numpy as np
import pytest

import oracle
import torchref
from bfhip import bfw


@pytest.fixture(scope="module")
def bev_model(tmp_path_factory):
    tensors = bfw.bev_stage_tensors(bfw._Init(2, "fan_in", 1.4))
    path = tmp_path_factory.mktemp("bev") / "bev.bfw"
    bfw.write_bfw(tensors, path)
    return path, dict(tensors)


@pytest.mark.parametrize("hw", [(8, 8), (6, 10)])
def test_bev_stage_bit_exact_with_reference_build(bev_model, hw):
    if not oracle.available("ref_scalar"):
        pytest.skip("reference CPU sources are not present to build oracle/_ref")
    path, _ = bev_model
    x = bfw.synthetic_bev(3, *hw)
    with oracle.scalar_env():
        outs = []
        for flavour in ("port_scalar", "ref_scalar"):
            o = oracle.Oracle(flavour)
            with o.open_model(path) as m:
                outs.append(o.bev_stage(m, x))
    for a, b in zip(*outs):
        assert a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_bev_stage_against_float64_torch(bev_model):
    path, p = bev_model
    x = bfw.synthetic_bev(4, 10, 14)
    o = oracle.Oracle("port")
    with o.open_model(path) as m:
        got = o.bev_stage(m, x)
    ref = torchref.bev_stage(p, x)
    for g, r, shape in zip(got, ref, ((1, 512, 10, 14), (1, 128, 10, 14), (1, 10, 10, 14))):
        assert g.shape == r.shape == shape
        scale = max(np.abs(r).max(), 1e-30)
        assert np.abs(g - r).max() <= 2e-5 * scale, np.abs(g - r).max() / scale


def test_bev_stage_rejections(bev_model):
    path, _ = bev_model
    o = oracle.Oracle("port")
    lib = o.lib
    h, w = 8, 8
    need = lib.bf_bev_stage_workspace_bytes(h, w)
    assert need == 2 * 256 * h * w * 4
    assert lib.bf_bev_stage_workspace_bytes(0, w) == 0
    x = bfw.synthetic_bev(0, h, w)
    sp = np.empty((1, 512, h, w), np.float32)
    sh = np.empty((1, 128, h, w), np.float32)
    hm = np.empty((1, 10, h, w), np.float32)
    ws = np.empty(need, np.uint8)
    err = C.create_string_buffer(256)
    with o.open_model(path) as m:
        net = m.create("bev_stage")
        try:
            assert lib.bf_bev_stage_forward_ref(net, x, 1, h, w, sp, sh, hm, ws.ctypes.data,
                                                need, err, 256)
            assert not lib.bf_bev_stage_forward_ref(net, x, 1, h, w, sp, sh, hm, ws.ctypes.data,
                                                    need - 1, err, 256)
            x7 = bfw.synthetic_bev(0, 7, 8)
            assert not lib.bf_bev_stage_forward_ref(net, x7, 1, 7, 8, sp, sh, hm,
                                                    ws.ctypes.data, need, err, 256)
            assert b"invalid" in err.value
        finally:
            lib.bf_bev_stage_destroy(net)
