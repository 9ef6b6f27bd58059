"""Integer index maps of the camera path, restated in numpy (TEST INFRASTRUCTURE ONLY).

Only ``tests/`` may import this module, as the checker of the device index
maps; nothing in the product path reads it.

* ``window_map``     padded, cyclically shifted window partition and the
                     shifted-window region labels: reference src/swin.c:106-117
                     (cyclic_source, mask_region) as used by the gather of
                     swin.c:119-219 and src/cuda_swin.cu:120-134.
* ``conv_im2col``    implicit-GEMM convolution addressing, direct and
                     transposed: reference src/cuda_ops.cu:23-56 (conv_input).

Pinned by tests/test_index_maps.py: the window map against a token-id grid
pushed through F.pad + torch.roll + window reshapes, the labels against the
slice-built region mask of mmdet's ShiftWindowMSA, and the im2col map against
the oracle's C convolution (bf_conv2d_f32_ref, bf_conv_transpose2d_f32_ref)
on random data.
"""

from __future__ import annotations

import numpy as np

WINDOW = 7


def window_map(batches: int, height: int, width: int, shift: int):
    """Return (token, label), both int32 [batches*wy*wx*49].

    token[w*49 + t] is the source row n*H*W + sy*W + sx of window token t, or
    -1 when the padded source lies outside the map.  label is 3*ry + rx of the
    padded position, region 0/1/2 = p < P-7 / p < P-shift / otherwise.
    """
    wy_n = -(-height // WINDOW)
    wx_n = -(-width // WINDOW)
    hp, wp = wy_n * WINDOW, wx_n * WINDOW
    n, wy, wx, t = np.meshgrid(np.arange(batches), np.arange(wy_n), np.arange(wx_n),
                               np.arange(49), indexing="ij")
    py = wy * WINDOW + t // WINDOW
    px = wx * WINDOW + t % WINDOW
    # swin.c:106-110 cyclic_source (forward direction).
    sy = (py + shift) % hp if shift else py
    sx = (px + shift) % wp if shift else px
    inside = (sy < height) & (sx < width)
    token = np.where(inside, (n * height + sy) * width + sx, -1)

    # swin.c:112-117 mask_region.
    def region(p, extent):
        return np.where(p < extent - WINDOW, 0, np.where(p < extent - shift, 1, 2))

    label = 3 * region(py, hp) + region(px, wp)
    return token.astype(np.int32).ravel(), label.astype(np.int32).ravel()


def conv_im2col(batches, ci, ih, iw, kh, kw, sh, sw, ph, pw, oh, ow, transpose):
    """Flat NCHW input index read at (row, reduction), or -1 for a zero tap.

    row = n*OH*OW + oy*OW + ox, reduction = ci*KH*KW + ky*KW + kx
    (src/cuda_ops.cu:23-56).  Returns int64 [rows, Ci*KH*KW].
    """
    rows = np.arange(batches * oh * ow)
    red = np.arange(ci * kh * kw)
    n = rows // (oh * ow)
    pos = rows - n * oh * ow
    oy, ox = pos // ow, pos % ow
    c = red // (kh * kw)
    kk = red - c * kh * kw
    ky, kx = kk // kw, kk % kw
    oy, ox, n = oy[:, None], ox[:, None], n[:, None]
    if not transpose:
        iy = oy * sh - ph + ky[None, :]
        ix = ox * sw - pw + kx[None, :]
        tap = np.ones(iy.shape, dtype=bool)
    else:
        sy = oy + ph - ky[None, :]
        sx = ox + pw - kx[None, :]
        tap = (sy >= 0) & (sx >= 0) & (sy % sh == 0) & (sx % sw == 0)
        iy = np.where(tap, sy // sh, -1)
        ix = np.where(tap, sx // sw, -1)
    inside = tap & (iy >= 0) & (iy < ih) & (ix >= 0) & (ix < iw)
    flat = ((n * ci + c[None, :]) * ih + iy) * iw + ix
    return np.where(inside, flat, -1).astype(np.int64)
