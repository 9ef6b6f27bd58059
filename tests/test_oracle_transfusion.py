"""CPU checks of the TransFusion oracle (oracle/src/transfusion.c).

Pinned by (a) the reference's own src/transfusion.c and
src/transfusion_decoder.c compiled as-is (oracle/_ref): bit-identical raw
outputs, labels and indices on the scalar path, and identical decoded
detections; (b) an independent float64 PyTorch restatement (F.max_pool2d
NMS, a stable descending torch.sort for the top-k,
F.multi_head_attention_forward for both attentions, F.conv1d position
embeddings and heads, F.layer_norm), so a wrong mask, tie rule, head split,
scale or residual fails; (c) known answers of the proposal selection (ties
broken by the smaller flat index, exempt classes 8/9, suppressed borders) and
the reference's rejections.
"""

import ctypes as C

import numpy as np
import pytest

import oracle
import torchref
from bfhip import bfw


@pytest.fixture(scope="module")
def tf_model(tmp_path_factory):
    tensors = bfw.transfusion_tensors(bfw._Init(3, "fan_in", 1.0))
    path = tmp_path_factory.mktemp("tf") / "tf.bfw"
    bfw.write_bfw(tensors, path)
    return path, dict(tensors)


@pytest.mark.parametrize("hw,proposals", [((12, 14), 20), ((20, 16), 64)])
def test_transfusion_bit_exact_with_reference_build(tf_model, hw, proposals):
    if not oracle.available("ref_scalar"):
        pytest.skip("reference CPU sources are not present to build oracle/_ref")
    path, _ = tf_model
    sh, hm = bfw.synthetic_transfusion_inputs(7, *hw)
    with oracle.scalar_env():
        res = []
        for flavour in ("port_scalar", "ref_scalar"):
            o = oracle.Oracle(flavour)
            with o.open_model(path) as m:
                outs = o.transfusion(m, sh, hm, proposals)
            res.append((outs, o.transfusion_detections(outs, 0.05)))
    (a, da), (b, db) = res
    for k in a:
        assert np.array_equal(a[k], b[k]), k
    assert len(da[0]) == len(db[0]) and np.array_equal(da[0], db[0])


@pytest.mark.parametrize("hw,proposals", [((16, 18), 40), ((2, 3), 60), ((1, 1), 10)])
def test_transfusion_against_float64_torch(tf_model, hw, proposals):
    """Includes proposals > H * W, where the reference's own workspace is too
    small for its self attention (the oracle sizes it by max(keys, P))."""
    path, p = tf_model
    sh, hm = bfw.synthetic_transfusion_inputs(8, *hw)
    o = oracle.Oracle("port")
    with o.open_model(path) as m:
        got = o.transfusion(m, sh, hm, proposals)
    ref = torchref.transfusion(p, sh, hm, proposals)
    assert np.array_equal(got["indices"], ref["indices"])
    assert np.array_equal(got["labels"], ref["labels"])
    for k, v in ref.items():
        if k in ("labels", "indices"):
            continue
        scale = max(np.abs(v).max(), 1e-30)
        assert np.abs(got[k] - v).max() <= 2e-5 * scale, (k, np.abs(got[k] - v).max() / scale)


def _select(o, logits, proposals):
    b, c, h, w = logits.shape
    sup = np.empty_like(logits)
    scores = np.empty((b, proposals), np.float32)
    cls = np.empty((b, proposals), np.int64)
    idx = np.empty((b, proposals), np.int64)
    ok = o.lib.bf_transfusion_select_proposals_f32_ref(logits, sup, scores, cls.ctypes.data,
                                                        idx.ctypes.data, b, c, h, w, proposals, 3)
    return ok, sup, scores, cls, idx


def test_proposal_selection_known_answers():
    o = oracle.Oracle("port")
    lg = np.full((1, 10, 5, 6), -30.0, np.float32)
    lg[0, 2, 2, 3] = 3.0      # interior maximum: kept
    lg[0, 2, 2, 2] = 1.0      # its neighbour: suppressed
    lg[0, 4, 0, 0] = 5.0      # border of an NMS class: suppressed
    lg[0, 8, 0, 0] = 2.0      # border of exempt class 8: kept
    lg[0, 9, 4, 5] = 3.0      # exempt class 9, same score as (2, 2, 3): later flat index
    lg[0, 5, 1, 1] = lg[0, 5, 1, 2] = 20.0  # two saturated neighbours (sigmoid 1.0): both kept
    ok, sup, scores, cls, idx = _select(o, np.ascontiguousarray(lg), 5)
    assert ok
    got = list(zip(cls[0].tolist(), idx[0].tolist()))
    assert got[:2] == [(5, 1 * 6 + 1), (5, 1 * 6 + 2)]   # equal 1.0 scores: smaller flat first
    assert got[2:4] == [(2, 2 * 6 + 3), (9, 4 * 6 + 5)]  # equal sigmoid(3): class 2 before 9
    assert got[4] == (8, 0)
    assert sup[0, 2, 2, 2] == 0.0 and sup[0, 4, 0, 0] == 0.0
    assert scores[0, 0] == 1.0 and scores[0, 2] == scores[0, 3]
    bad = np.zeros((1, 10, 4, 4), np.float32)
    assert not _select(o, bad, 0)[0]
    assert not _select(o, bad, 201)[0]


def test_decoder_rejections(tf_model):
    path, _ = tf_model
    o = oracle.Oracle("port")
    lib = o.lib
    need = lib.bf_transfusion_decoder_workspace_bytes(12, 14, 20)
    assert need == 4 * (168 * (3 * 128 + 10 + 16) + 20 * (8 * 128 + 1))
    # Projection and score-slot rows are max(keys, proposals).
    assert lib.bf_transfusion_decoder_workspace_bytes(2, 3, 60) == 4 * (
        6 * (128 + 10) + 60 * (2 * 128 + 16) + 60 * (8 * 128 + 1))
    assert lib.bf_transfusion_decoder_workspace_bytes(12, 14, 201) == 0
    assert lib.bf_transfusion_decoder_workspace_bytes(1, 1, 11) == 0
    sh, hm = bfw.synthetic_transfusion_inputs(0, 12, 14)
    outs = {k: np.empty((1, c, 20), np.float32) for k, c in o.TF_FIELDS}
    labels, indices = np.empty((1, 20), np.int64), np.empty((1, 20), np.int64)
    raw = oracle.TfRaw(*[outs[k].ctypes.data for k, _ in o.TF_FIELDS], labels.ctypes.data,
                       indices.ctypes.data)
    ws = np.empty(need, np.uint8)
    err = C.create_string_buffer(256)
    with o.open_model(path) as m:
        net = m.create("transfusion_decoder")
        try:
            assert lib.bf_transfusion_decoder_forward_ref(net, sh, hm, 1, 12, 14, 20, C.byref(raw),
                                                          ws.ctypes.data, need, err, 256)
            assert not lib.bf_transfusion_decoder_forward_ref(
                net, sh, hm, 1, 12, 14, 20, C.byref(raw), ws.ctypes.data, need - 1, err, 256)
            assert b"invalid" in err.value
        finally:
            lib.bf_transfusion_decoder_destroy(net)
