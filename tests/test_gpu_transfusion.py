"""TransFusion decoder context on the GPU (include/bf_cuda_transfusion.h)
against the CPU oracle (oracle/src/transfusion.c, itself pinned bit-exact to
the reference build and to a float64 torch restatement).

Follows the reference's tests/test_cuda_transfusion.cu: the raw outputs of
one forward against the CPU decoder, a repeat, and the decoded detections.
Bars: proposal labels, indices and the NMS'd query scores bit-exact (the
scores are the reference's two-branch logistic with a correctly rounded exp,
so the selection is the same total order); every floating-point field within
the north-star tolerance (rel-L2 <= 1e-2, max-abs <= 5e-2 RMS, tests/util.py)
-- the key side and the cross attention run fp16 operands with fp32
accumulation.  Shapes cover a single cell, every candidate selected
(zero-score ties), key counts that are not a multiple of the 64-key step, and
the production 180 x 180 map with 200 proposals (64 key splits).
"""

import numpy as np
import pytest

import bfhip
import oracle
from bfhip import bfw
from util import assert_close

pytestmark = pytest.mark.gpu

FLOAT_FIELDS = [k for k, _ in bfhip.TF_FIELDS if k != "query_scores"]


@pytest.fixture(scope="module")
def tf_path(tmp_path_factory):
    return bfw.write_transfusion(tmp_path_factory.mktemp("tf") / "tf.bfw", seed=3,
                                 mode="fan_in", gain=1.0)


def _gpu(path, shared, heatmap, proposals, device):
    import torch
    with bfhip.Model(path) as m:
        dec = bfhip.TransFusion(m, shared.shape[2], shared.shape[3], proposals)
    sh = torch.from_numpy(shared).to(device)
    hm = torch.from_numpy(heatmap).to(device)
    print(f"[case] transfusion {shared.shape[2]}x{shared.shape[3]} P={proposals}", flush=True)
    outs = dec.forward(sh, hm)
    again = dec.forward(sh, hm)
    torch.cuda.synchronize()
    got = {k: v.cpu().numpy() for k, v in outs.items()}
    for k, v in again.items():
        assert np.array_equal(got[k], v.cpu().numpy()), f"{k}: forward is not repeatable"
    assert dec.resident_bytes() > 0
    return dec, outs, got


def _oracle(path, shared, heatmap, proposals):
    o = oracle.Oracle("port")
    with o.open_model(path) as m:
        return o, o.transfusion(m, shared, heatmap, proposals)


def _check(got, want, tag):
    assert np.array_equal(got["labels"], want["labels"]), f"{tag}: labels differ"
    assert np.array_equal(got["indices"], want["indices"]), f"{tag}: indices differ"
    assert np.array_equal(got["query_scores"], want["query_scores"]), f"{tag}: query scores differ"
    for k in FLOAT_FIELDS:
        assert got[k].shape == want[k].shape, k
        assert_close(got[k], want[k], f"transfusion {k} {tag}")


@pytest.mark.parametrize("hw,proposals", [((1, 1), 10), ((2, 3), 60), ((12, 14), 20),
                                          ((20, 16), 64), ((36, 52), 200), ((180, 180), 200)])
def test_transfusion_matches_oracle(tf_path, hw, proposals, device):
    sh, hm = bfw.synthetic_transfusion_inputs(11, *hw)
    dec, _, got = _gpu(tf_path, sh, hm, proposals, device)
    _, want = _oracle(tf_path, sh, hm, proposals)
    _check(got, want, f"{hw} P={proposals}")
    dec.close()


@pytest.mark.parametrize("kind", ["constant", "integer"])
def test_transfusion_selection_ties(tf_path, kind, device):
    """Exact score ties are broken by the smaller flat index: a constant map
    (every interior cell of classes 0-7 survives NMS with the same score)
    and integer-quantised logits (many equal scores)."""
    sh, hm = bfw.synthetic_transfusion_inputs(12, 24, 20)
    if kind == "constant":
        hm = np.full_like(hm, 0.75)
    else:
        hm = np.round(hm * 2.0).astype(np.float32)
    dec, _, got = _gpu(tf_path, sh, hm, 200, device)
    _, want = _oracle(tf_path, sh, hm, 200)
    _check(got, want, kind)
    dec.close()


@pytest.mark.parametrize("kind", ["constant", "flat"])
def test_transfusion_selection_many_candidates(tf_path, kind, device):
    """Production map with far more candidates past the first radix digit
    than the one-workgroup finish holds in LDS (8192), so it reads them in
    place: every cell at one score (324 000 exact ties), and the flat
    heatmap of random weights (logits -1 +- 0.05, scores 0.26-0.28, as in
    the runtime's synthetic frames)."""
    sh, hm = bfw.synthetic_transfusion_inputs(15, 180, 180)
    if kind == "constant":
        hm = np.full_like(hm, 0.75)
    else:
        hm = (-1.0 + 0.05 * np.random.default_rng(15).standard_normal(hm.shape)).astype(np.float32)
    dec, _, got = _gpu(tf_path, sh, hm, 200, device)
    _, want = _oracle(tf_path, sh, hm, 200)
    _check(got, want, kind)
    dec.close()


def test_transfusion_decode_matches_oracle(tf_path, device):
    """GPU decode + filter of one forward's raw outputs against the oracle's
    decode_raw + filter of the same outputs: same kept set and order, class
    ids exact, boxes within a few ulps (device expf / atan2f)."""
    sh, hm = bfw.synthetic_transfusion_inputs(13, 36, 52)
    dec, outs, got = _gpu(tf_path, sh, hm, 200, device)
    o = oracle.Oracle("port")
    for threshold in (-1.0, 0.05, 0.2, 2.0):
        dets = dec.decode(outs, threshold)
        g = oracle.detections_array(dets)
        w = o.transfusion_detections(got, threshold)[0]
        assert g.shape == w.shape, f"threshold {threshold}: {g.shape} vs {w.shape}"
        assert np.array_equal(g[:, 10], w[:, 10])
        np.testing.assert_allclose(g[:, :10], w[:, :10], rtol=2e-6, atol=1e-6)
    assert dec.decode(outs, 2.0).count == 0
    dec.close()


def test_transfusion_graph_replays(tf_path, device):
    import torch
    sh, hm = bfw.synthetic_transfusion_inputs(14, 36, 52)
    dec, outs, eager = _gpu(tf_path, sh, hm, 200, device)
    shd, hmd = torch.from_numpy(sh).to(device), torch.from_numpy(hm).to(device)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        dec.forward(shd, hmd, outs, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dec.forward(shd, hmd, outs)
    for i in range(3):
        for v in outs.values():
            v.fill_(i + 1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k, v in outs.items():
            assert np.array_equal(v.cpu().numpy(), eager[k]), f"replay {i}: {k} differs"
    dec.close()
