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
