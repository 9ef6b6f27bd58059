"""Integer index maps of the camera path, restated in numpy (TEST INFRASTRUCTURE ONLY).

Only ``tests/`` may import this module, as the checker of the device index
maps; nothing in the product path reads it.

* ``window_map``     padded, cyclically shifted window partition and the
                     shifted-window region labels: reference src/swin.c:106-117
                     (cyclic_source, mask_region) as used by the gather of
                     swin.c:119-219 and src/cuda_swin.cu:120-134.
* ``conv_im2col``    implicit-GEMM convolution addressing, direct and
                     transposed: reference src/cuda_ops.cu:23-56 (conv_input).
* ``conv_im2col_nhwc`` the same addressing over a channels-last map, with the
                     reduction ordered tap-major (k = (ky*KW + kx)*Ci + c) and
                     optionally the output pixels x-major: the element the
                     reference's conv_input reads for input channel c and
                     tap (ky, kx), in the layout the camera neck's GEMMs use.
* ``merge_unfold``   Swin patch-merge unfold: reference src/swin_backbone.c:
                     278-302 (nn.Unfold order c*4 + ky*2 + kx, zero past an odd
                     edge) and src/cuda_swin.cu:218-225.
* ``bilinear_taps`` / ``bilinear_onehot``  FPN bilinear upsampling
                     (align_corners = False) in the reference's float32
                     operation order: src/image_fpn.c:123-142
                     (bilinear_channel).

Pinned by tests/test_index_maps.py: the window map against a token-id grid
pushed through F.pad + torch.roll + window reshapes, the labels against the
slice-built region mask of mmdet's ShiftWindowMSA, the im2col map against
the oracle's C convolution (bf_conv2d_f32_ref, bf_conv_transpose2d_f32_ref)
on random data, the channels-last map against the NCHW map (same elements
after the layout change, and the conv of random data it implies against
torch), the unfold against F.pad + F.unfold, and the bilinear taps against
F.interpolate (bilinear, align_corners = False) in float64 and, for the
dyadic 2x case, exactly.
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


def conv_im2col_nhwc(batches, ci, ih, iw, kh, kw, sh, sw, ph, pw, oh, ow, yfast=False,
                     rows=None):
    """Flat channels-last input index ((n*IH + iy)*IW + ix)*Ci + c read at
    (row, k), k = (ky*KW + kx)*Ci + c, or -1 for a tap outside the map: the
    element reference conv_input (src/cuda_ops.cu:23-56) reads for output
    pixel (oy, ox), input channel c and tap (ky, kx), iy = oy*SH - PH + ky,
    ix = ox*SW - PW + kx.  Rows are n*OH*OW + oy*OW + ox, or with yfast
    n*OH*OW + ox*OH + oy; `rows` (a range) selects a slice of them.
    Returns int64 [len(rows), KH*KW*Ci]."""
    rows = np.arange(batches * oh * ow) if rows is None else np.asarray(rows)
    n = rows // (oh * ow)
    pos = rows - n * oh * ow
    if yfast:
        ox, oy = pos // oh, pos % oh
    else:
        oy, ox = pos // ow, pos % ow
    k = np.arange(kh * kw * ci)
    tap, c = k // ci, k % ci
    ky, kx = tap // kw, tap % kw
    iy = oy[:, None] * sh - ph + ky[None, :]
    ix = ox[:, None] * sw - pw + kx[None, :]
    inside = (iy >= 0) & (iy < ih) & (ix >= 0) & (ix < iw)
    flat = ((n[:, None] * ih + iy) * iw + ix) * ci + c[None, :]
    return np.where(inside, flat, -1).astype(np.int64)


def merge_unfold(batches, height, width, channels):
    """Flat token-channel index ((n*H + y)*W + x)*C + c of the Swin patch-merge
    unfold row m = (n, oy, ox) at column c*4 + ky*2 + kx (y = 2*oy + ky,
    x = 2*ox + kx), or -1 past an odd edge (src/swin_backbone.c:278-302).
    Returns int64 [batches*H2*W2, 4*C]."""
    h2, w2 = -(-height // 2), -(-width // 2)
    m = np.arange(batches * h2 * w2)
    n, p = m // (h2 * w2), m % (h2 * w2)
    oy, ox = p // w2, p % w2
    col = np.arange(4 * channels)
    c, q = col // 4, col % 4
    ky, kx = q // 2, q % 2
    y = 2 * oy[:, None] + ky[None, :]
    x = 2 * ox[:, None] + kx[None, :]
    inside = (y < height) & (x < width)
    flat = ((n[:, None] * height + y) * width + x) * channels + c[None, :]
    return np.where(inside, flat, -1).astype(np.int64)


def bilinear_taps(in_h, in_w, out_h, out_w):
    """Per output row y and column x: (y0, y1, fy) and (x0, x1, fx) of
    src/image_fpn.c:123-142 in float32, operation by operation:
    source = ((float)y + 0.5f) * (float)in / (float)out - 0.5f, clamped below
    at 0; y0 = floor, y1 = y0 + 1 if inside else y0; fy = source - y0."""
    f = np.float32

    def axis(inn, out):
        o = np.arange(out).astype(f)
        src = (o + f(0.5)) * f(inn) / f(out) - f(0.5)
        src = np.where(src < f(0.0), f(0.0), src).astype(f)
        i0 = np.floor(src).astype(np.int64)
        i1 = np.where(i0 + 1 < inn, i0 + 1, i0)
        frac = (src - i0.astype(f)).astype(f)
        return i0, i1, frac

    return axis(in_h, out_h), axis(in_w, out_w)


def bilinear_onehot(in_h, in_w, out_h, out_w, select):
    """Bilinear upsampling (src/image_fpn.c:123-142, float32, the reference's
    operation order) of one-hot maps: map j is 1 at source pixel select[j]
    (flat y*in_w + x) and 0 elsewhere.  Returns float32 [len(select), out_h,
    out_w]: the weight each output pixel gives that source pixel."""
    f = np.float32
    (y0, y1, fy), (x0, x1, fx) = bilinear_taps(in_h, in_w, out_h, out_w)
    sel = np.asarray(select, np.int64)
    sy, sx = (sel // in_w)[:, None, None], (sel % in_w)[:, None, None]
    Y0, Y1, FY = y0[None, :, None], y1[None, :, None], fy[None, :, None]
    X0, X1, FX = x0[None, None, :], x1[None, None, :], fx[None, None, :]
    one = f(1.0)
    a = ((Y0 == sy) & (X0 == sx)).astype(f)
    b = ((Y0 == sy) & (X1 == sx)).astype(f)
    c = ((Y1 == sy) & (X0 == sx)).astype(f)
    d = ((Y1 == sy) & (X1 == sx)).astype(f)
    top = (a * (one - FX)).astype(f) + (b * FX).astype(f)
    bottom = (c * (one - FX)).astype(f) + (d * FX).astype(f)
    return ((top * (one - FY)).astype(f) + (bottom * FY).astype(f)).astype(f)
