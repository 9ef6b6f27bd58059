"""Pin oracle/index_maps.py, the integer maps the device index tests check
against (CPU only).

* Window partition: a grid of token ids is zero-padded (here: -1) with F.pad,
  rolled by -shift with torch.roll and cut into 7x7 windows with reshapes, the
  construction of mmdet's ShiftWindowMSA; the oracle's closed form must give
  the same ids in the same order.
* Region labels: the img_mask of ShiftWindowMSA, built from the three slices
  (0, -7), (-7, -shift), (-shift, None) per axis, then window-partitioned.
* im2col: the gathered matrix times the weights must equal the oracle's C
  convolution (bf_conv2d_f32_ref / bf_conv_transpose2d_f32_ref) on random data.
"""

import numpy as np
import pytest

import oracle
from oracle import index_maps

OR = oracle.Oracle("port")

WINDOW_SHAPES = [(1, 7, 7), (2, 5, 7), (1, 9, 12), (2, 64, 176), (1, 32, 88), (1, 16, 44),
                 (3, 8, 22), (1, 3, 4)]


def torch_windows(grid, shift):
    import torch
    import torch.nn.functional as F
    t = torch.from_numpy(grid)
    b, h, w = t.shape
    hp, wp = -(-h // 7) * 7, -(-w // 7) * 7
    t = F.pad(t, (0, wp - w, 0, hp - h), value=-1)
    if shift:
        t = torch.roll(t, shifts=(-shift, -shift), dims=(1, 2))
    t = t.view(b, hp // 7, 7, wp // 7, 7).permute(0, 1, 3, 2, 4).reshape(-1)
    return t.numpy()


@pytest.mark.parametrize("shape", WINDOW_SHAPES)
@pytest.mark.parametrize("shift", [0, 3, 1])
def test_window_tokens_match_pad_roll_partition(shape, shift):
    b, h, w = shape
    ids = np.arange(b * h * w, dtype=np.int64).reshape(b, h, w)
    expect = torch_windows(ids, shift)
    token, _ = index_maps.window_map(b, h, w, shift)
    np.testing.assert_array_equal(token, expect)


@pytest.mark.parametrize("shape", WINDOW_SHAPES)
@pytest.mark.parametrize("shift", [3, 1, 2])
def test_window_labels_match_slice_mask(shape, shift):
    b, h, w = shape
    hp, wp = -(-h // 7) * 7, -(-w // 7) * 7
    mask = np.zeros((hp, wp), np.int64)
    cnt = 0
    slices = (slice(0, -7), slice(-7, -shift), slice(-shift, None))
    for hs in slices:
        for ws in slices:
            mask[hs, ws] = cnt
            cnt += 1
    expect = mask.reshape(hp // 7, 7, wp // 7, 7).transpose(0, 2, 1, 3).reshape(-1)
    expect = np.tile(expect, b)
    _, label = index_maps.window_map(b, h, w, shift)
    np.testing.assert_array_equal(label, expect)


def test_unshifted_padded_keys_are_kept():
    """shift 0: padded tokens are present (-1) but never separated by labels
    (the reference masks nothing in regular blocks, swin.c:190)."""
    token, _ = index_maps.window_map(1, 9, 12, 0)
    assert (token == -1).sum() == 14 * 14 - 9 * 12


CONV_CASES = [
    # batches, Ci, IH, IW, KH, KW, SH, SW, PH, PW, OH, OW, transpose
    (2, 3, 6, 7, 3, 3, 2, 2, 1, 1, 3, 4, 0),
    (1, 2, 9, 10, 5, 5, 4, 4, 2, 2, 3, 3, 0),
    (1, 3, 4, 6, 2, 2, 2, 2, 0, 0, 8, 12, 1),
    (1, 4, 5, 5, 3, 3, 2, 2, 1, 1, 9, 9, 1),
    (1, 7, 21, 19, 5, 5, 2, 2, 2, 2, 11, 10, 0),
    (2, 5, 8, 8, 1, 1, 1, 1, 0, 0, 8, 8, 0),
]


@pytest.mark.parametrize("case", CONV_CASES)
def test_im2col_times_weights_is_the_oracle_conv(case):
    n, ci, ih, iw, kh, kw, sh, sw, ph, pw, oh, ow, tr = case
    r = np.random.default_rng(7)
    co = 5
    x = r.standard_normal((n, ci, ih, iw)).astype(np.float32)
    idx = index_maps.conv_im2col(n, ci, ih, iw, kh, kw, sh, sw, ph, pw, oh, ow, tr)
    cols = np.where(idx >= 0, x.reshape(-1)[np.maximum(idx, 0)], 0.0)
    if tr:
        w = r.standard_normal((ci, co, kh, kw)).astype(np.float32)
        wm = w.transpose(1, 0, 2, 3).reshape(co, -1)
        ref = OR.conv_transpose2d(x, w, None, stride=(sh, sw), pad=(ph, pw))
    else:
        w = r.standard_normal((co, ci, kh, kw)).astype(np.float32)
        wm = w.reshape(co, -1)
        ref = OR.conv2d(x, w, None, (sh, sw), (ph, pw), scalar=True)
    got = (cols.astype(np.float64) @ wm.T.astype(np.float64)).reshape(n, oh, ow, co)
    got = got.transpose(0, 3, 1, 2)
    assert ref.shape == got.shape
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


# Channels-last gather map: the camera neck's geometries (batch 2) plus odd
# sizes, strides and the x-major row order.
NHWC_GEOMS = [
    # (ci, ih, iw, k, stride, pad)
    (16, 16, 44, 3, 1, 1), (8, 64, 176, 5, 4, 2), (32, 64, 176, 5, 2, 2), (24, 32, 88, 1, 1, 0),
    (16, 36, 36, 3, 2, 1), (8, 5, 7, 3, 1, 1), (8, 7, 5, 5, 2, 2),
]


@pytest.mark.parametrize("geom", NHWC_GEOMS)
@pytest.mark.parametrize("yfast", [False, True])
def test_conv_im2col_nhwc_is_the_nchw_map_relaid(geom, yfast):
    ci, ih, iw, k, s, p = geom
    b = 2
    oh, ow = (ih + 2 * p - k) // s + 1, (iw + 2 * p - k) // s + 1
    nchw = index_maps.conv_im2col(b, ci, ih, iw, k, k, s, s, p, p, oh, ow, False)
    nhwc = index_maps.conv_im2col_nhwc(b, ci, ih, iw, k, k, s, s, p, p, oh, ow, yfast)
    # NCHW flat -> (n, c, iy, ix) -> NHWC flat; reduction c*KK + tap -> tap*Ci + c.
    n = nchw // (ci * ih * iw)
    r = nchw % (ci * ih * iw)
    c, iy, ix = r // (ih * iw), (r // iw) % ih, r % iw
    relaid = np.where(nchw >= 0, ((n * ih + iy) * iw + ix) * ci + c, -1)
    kk = k * k
    col = np.arange(kk * ci)
    relaid = relaid[:, (col % ci) * kk + col // ci]
    if yfast:  # GEMM row n*OH*OW + ox*OH + oy holds NCHW row n*OH*OW + oy*OW + ox
        rows = np.arange(b * oh * ow)
        nn, pos = rows // (oh * ow), rows % (oh * ow)
        relaid = relaid[nn * oh * ow + (pos % oh) * ow + pos // oh]
    np.testing.assert_array_equal(nhwc, relaid)
    part = index_maps.conv_im2col_nhwc(b, ci, ih, iw, k, k, s, s, p, p, oh, ow, yfast,
                                       rows=range(5, 17))
    np.testing.assert_array_equal(part, nhwc[5:17])


@pytest.mark.parametrize("geom", NHWC_GEOMS[:4])
def test_conv_im2col_nhwc_gathers_torch_conv(geom):
    """The gathered rows times channels-last weights are torch's conv2d."""
    import torch
    import torch.nn.functional as F
    ci, ih, iw, k, s, p = geom
    b, co = 2, 5
    oh, ow = (ih + 2 * p - k) // s + 1, (iw + 2 * p - k) // s + 1
    rng = np.random.default_rng(7)
    x = rng.standard_normal((b, ih, iw, ci))
    w = rng.standard_normal((co, ci, k, k))
    idx = index_maps.conv_im2col_nhwc(b, ci, ih, iw, k, k, s, s, p, p, oh, ow)
    flat = np.concatenate([x.ravel(), [0.0]])
    a = flat[np.where(idx >= 0, idx, flat.size - 1)]
    got = a @ w.transpose(0, 2, 3, 1).reshape(co, -1).T
    ref = F.conv2d(torch.from_numpy(x).permute(0, 3, 1, 2), torch.from_numpy(w), stride=s,
                   padding=p).permute(0, 2, 3, 1).reshape(-1, co).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("shape", [(2, 8, 22, 3), (1, 7, 14, 4), (2, 5, 7, 2), (1, 1, 1, 8),
                                   (1, 64, 176, 2)])
def test_merge_unfold_matches_pad_unfold(shape):
    import torch
    import torch.nn.functional as F
    b, h, w, c = shape
    ids = np.arange(b * h * w * c, dtype=np.float64).reshape(b, h, w, c) + 1
    t = torch.from_numpy(ids).permute(0, 3, 1, 2)
    t = F.pad(t, (0, w % 2, 0, h % 2))
    u = F.unfold(t, kernel_size=2, stride=2)  # [b, 4c, L], rows c*4 + ky*2 + kx
    expect = u.permute(0, 2, 1).reshape(-1, 4 * c).numpy().astype(np.int64) - 1
    np.testing.assert_array_equal(index_maps.merge_unfold(b, h, w, c), expect)


@pytest.mark.parametrize("sizes", [(16, 44, 32, 88), (8, 22, 16, 44), (3, 4, 5, 7), (2, 2, 3, 4),
                                   (5, 3, 9, 6), (1, 1, 2, 2)])
def test_bilinear_onehot_matches_interpolate(sizes):
    import torch
    import torch.nn.functional as F
    ih, iw, oh, ow = sizes
    sel = np.arange(ih * iw)
    got = index_maps.bilinear_onehot(ih, iw, oh, ow, sel)
    eye = torch.eye(ih * iw, dtype=torch.float64).reshape(ih * iw, 1, ih, iw)
    ref = F.interpolate(eye, size=(oh, ow), mode="bilinear", align_corners=False)[:, 0].numpy()
    np.testing.assert_allclose(got, ref, rtol=0, atol=2e-7)
    if oh == 2 * ih and ow == 2 * iw:  # dyadic weights: exact in float32
        np.testing.assert_array_equal(got, ref.astype(np.float32))
