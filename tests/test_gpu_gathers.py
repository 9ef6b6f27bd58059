"""Bit-exact integer work of the production gathers, through the probes of
include/bfhip_debug.h, against oracle/index_maps.py (pinned on the CPU by
tests/test_index_maps.py).

* Camera-neck convs (bfhip_debug_camera_gather): each layer's A-operand gather
  runs with the tile, pipeline and loader instance of the forward over
  identity weights, so the fp32 output is the gathered operand.  Inputs are
  1 + base-2047 digits of the element's pixel index, or 1 + its channel, in
  three passes (each value exact in fp16), which decode to the (pixel,
  channel) every tap read; zero marks a tap outside the map.  Covered: the
  single-source LDS-DMA gathers (fpn_convs.0/.1, depthnet.3, dtransform.6),
  the two-source concat of depthnet.0, the 1x1 of depthnet.6, the
  96-channel-stride downsample rows (stride 1 and 2) and the x-major
  (transposed-store) rows of the last downsample conv, and the register-fed
  dtransform.3 gather with dtransform.0's affine evaluated in it (depth
  digits d in [1, 256], affine d + 256 c: exact, decodes to pixel and
  virtual channel).
* Swin patch merges (bfhip_debug_swin_merge_gather): the tap-major 2x2 token
  gather composed with the create-time column permutation reproduces the
  reference's unfold matrix, odd edges included.
* FPN upsampling (bfhip_debug_fpn_upsample): the lateral convs' epilogue over
  a zero product, on one-hot upper maps (one source pixel per channel), gives
  every bilinear weight; with 0/1 inputs each product is exact, so the fp16
  outputs must equal the oracle's float32 bilinear_channel restatement bit for
  bit, clamped borders and non-dyadic ratios included.

Production shapes: neck at 6 x 32 x 88 features (256 x 704 depth) and a
360 x 360 BEV; Swin at 6 x 256 x 704.  Odd shapes: neck at 2 x 5 x 7 with a
12 x 6 BEV, Swin at 2 x 56 x 112.
"""

import numpy as np
import pytest

from oracle import index_maps

pytestmark = pytest.mark.gpu

BASE = 2047  # 1 + digit stays <= 2048: exact in fp16

# layer -> (kernel, stride, pad, yfast)
CONV = {1: (3, 1, 1, False), 3: (3, 1, 1, False), 4: (5, 4, 2, False), 5: (5, 2, 2, False),
        6: (3, 1, 1, False), 7: (3, 1, 1, False), 8: (1, 1, 0, False), 9: (3, 1, 1, False),
        10: (3, 2, 1, False), 11: (3, 1, 1, True)}


def _neck(tmp_models, b, h, w, bev):
    import bfhip
    with bfhip.Model(tmp_models()) as m:
        return bfhip.CameraNeck(m, b, h, w, bev[0], bev[1])


def _input_shape(layer, b, h, w, bev):
    """(batch, IH, IW, channels) of the layer's channels-last input."""
    h1, w1 = -(-h // 2), -(-w // 2)
    return {1: (b, h1, w1, 256), 3: (b, h, w, 256), 4: (b, 8 * h, 8 * w, 8),
            5: (b, 2 * h, 2 * w, 32), 6: (b, h, w, 320), 7: (b, h, w, 256),
            8: (b, h, w, 256), 9: (1, bev[0], bev[1], 96), 10: (1, bev[0], bev[1], 96),
            11: (1, bev[0] // 2, bev[1] // 2, 96)}[layer]


def _digit_maps(n, ih, iw, ci, device):
    """The three encodings of a channels-last map: pixel digit 0, pixel digit
    1, channel (each 1 + value, fp16)."""
    import torch
    pix = torch.arange(n * ih * iw, device=device, dtype=torch.int64).view(n, ih, iw, 1)
    chan = torch.arange(ci, device=device, dtype=torch.int64).view(1, 1, 1, ci)
    out = []
    for v in (pix % BASE, pix // BASE, chan):
        out.append((1 + v).expand(n, ih, iw, ci).to(torch.float16).contiguous())
    return out


def _compare_chunked(idx, expect_rows, rows=4096):
    m = idx.shape[0]
    for r0 in range(0, m, rows):
        r1 = min(m, r0 + rows)
        got = idx[r0:r1].cpu().numpy()
        exp = expect_rows(range(r0, r1))
        if not np.array_equal(got, exp):
            bad = np.argwhere(got != exp)[0]
            raise AssertionError(f"row {r0 + bad[0]} col {bad[1]}: read {got[tuple(bad)]}, "
                                 f"oracle {exp[tuple(bad)]}")


def _gather_conv(neck, layer, shape, device):
    """Decoded flat channels-last index [M, K] (int64, -1 outside) of every
    element the layer's gather reads."""
    import torch
    import bfhip
    n, ih, iw, ci = shape
    if layer == 4:
        pix = torch.arange(n * ih * iw, device=device, dtype=torch.int64).view(n, ih, iw)
        affine = torch.tensor([1.0] * 8 + [256.0 * c for c in range(8)], device=device)
        digits, chans = [], []
        for j in range(3):
            d = (1 + (pix >> (8 * j)) % 256).to(torch.float32).contiguous()
            v = bfhip.camera_gather(neck, 4, d, affine=affine).to(torch.int64)
            valid = v > 0
            digits.append(torch.where(valid, (v - 1) % 256, 0))
            chans.append(torch.where(valid, (v - 1) // 256, -1))
        assert torch.equal(chans[0], chans[1]) and torch.equal(chans[0], chans[2])
        flat = (digits[0] + (digits[1] << 8) + (digits[2] << 16)) * 8 + chans[0]
        return torch.where(chans[0] >= 0, flat, -1)
    if layer == 6:
        maps0 = _digit_maps(n, ih, iw, 64, device)
        maps1 = _digit_maps(n, ih, iw, 256, device)
        maps1[2] = (maps1[2].float() + 64).half().contiguous()  # concat channel 64 + c
        outs = [bfhip.camera_gather(neck, 6, a, b).to(torch.int64) for a, b in zip(maps0, maps1)]
    else:
        outs = [bfhip.camera_gather(neck, layer, a).to(torch.int64)
                for a in _digit_maps(n, ih, iw, ci, device)]
    valid = outs[0] > 0
    assert torch.equal(valid, outs[1] > 0) and torch.equal(valid, outs[2] > 0)
    flat = ((outs[0] - 1) + BASE * (outs[1] - 1)) * ci + (outs[2] - 1)
    return torch.where(valid, flat, -1)


NECK_SHAPES = {"production": (6, 32, 88, (360, 360)), "odd": (2, 5, 7, (12, 6))}


@pytest.mark.parametrize("shape", ["production", "odd"])
@pytest.mark.parametrize("layer", sorted(CONV))
def test_camera_conv_gather_bit_exact(device, tmp_models, shape, layer):
    import torch
    b, h, w, bev = NECK_SHAPES[shape]
    print(f"camera gather: layer {layer}, {shape} {b}x{h}x{w} bev {bev}", flush=True)
    neck = _neck(tmp_models, b, h, w, bev)
    try:
        n, ih, iw, ci = _input_shape(layer, b, h, w, bev)
        k, s, p, yfast = CONV[layer]
        oh, ow = (ih + 2 * p - k) // s + 1, (iw + 2 * p - k) // s + 1
        idx = _gather_conv(neck, layer, (n, ih, iw, ci), device)
        torch.cuda.synchronize()
        assert tuple(idx.shape) == (n * oh * ow, k * k * ci)
        _compare_chunked(idx, lambda rows: index_maps.conv_im2col_nhwc(
            n, ci, ih, iw, k, k, s, s, p, p, oh, ow, yfast, rows=rows))
    finally:
        neck.close()


SWIN_SHAPES = {"production": (6, 256, 704), "odd": (2, 56, 112)}


@pytest.mark.parametrize("shape", ["production", "odd"])
@pytest.mark.parametrize("stage", [0, 1, 2])
def test_swin_merge_gather_bit_exact(device, tmp_models, shape, stage):
    import torch
    import bfhip
    b, hi, wi = SWIN_SHAPES[shape]
    print(f"merge gather: stage {stage}, {shape} {b}x{hi}x{wi}", flush=True)
    with bfhip.Model(tmp_models()) as m:
        swin = bfhip.Swin(m, b, hi, wi)
    try:
        h, w = -(-hi // 4), -(-wi // 4)
        for _ in range(stage):
            h, w = -(-h // 2), -(-w // 2)
        c = (96, 192, 384)[stage]
        outs = [bfhip.swin_merge_gather(swin, stage, x).to(torch.int64)
                for x in _digit_maps(b, h, w, c, device)]
        valid = outs[0] > 0
        assert torch.equal(valid, outs[1] > 0) and torch.equal(valid, outs[2] > 0)
        flat = ((outs[0] - 1) + BASE * (outs[1] - 1)) * c + (outs[2] - 1)
        got = torch.where(valid, flat, -1).cpu().numpy()
        np.testing.assert_array_equal(got, index_maps.merge_unfold(b, h, w, c))
        if h % 2 or w % 2:
            assert (got == -1).any()
    finally:
        swin.close()


@pytest.mark.parametrize("shape", ["production", "odd"])
@pytest.mark.parametrize("level", [0, 1])
def test_fpn_upsample_bit_exact(device, tmp_models, shape, level):
    import torch
    import bfhip
    b, h, w, bev = NECK_SHAPES[shape]
    print(f"fpn upsample: level {level}, {shape} {b}x{h}x{w}", flush=True)
    neck = _neck(tmp_models, b, h, w, bev)
    try:
        h1, w1 = -(-h // 2), -(-w // 2)
        h2, w2 = -(-h1 // 2), -(-w1 // 2)
        (H, W), (hu, wu) = ((h, w), (h1, w1)) if level == 0 else ((h1, w1), (h2, w2))
        for q in range(-(-hu * wu // 256)):
            sel = (q * 256 + np.arange(256)[None, :] + 97 * np.arange(b)[:, None]) % (hu * wu)
            up = np.zeros((b, hu * wu, 256), np.float32)
            up[np.arange(b)[:, None], sel, np.arange(256)[None, :]] = 1.0
            got = bfhip.fpn_upsample(neck, level, torch.from_numpy(up.reshape(b, hu, wu, 256))
                                     .to(device))
            weights = index_maps.bilinear_onehot(hu, wu, H, W, sel.ravel())  # [b*256, H, W]
            expect = weights.reshape(b, 256, H, W).transpose(0, 2, 3, 1).astype(np.float16)
            np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16), expect.view(np.uint16))
    finally:
        neck.close()
