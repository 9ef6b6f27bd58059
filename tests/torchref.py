"""Independent float64 PyTorch restatements of the path's semantics.

Written from the mmdet / mmcv module semantics the reference checkpoint comes
from (ShiftWindowMSA with pad-then-roll and a -100 region mask, PatchMerging
through nn.Unfold, GeneralizedLSSFPN bilinear upsampling with
align_corners=False), using library routines (torch.roll, F.pad, F.unfold,
F.interpolate, F.layer_norm, F.gelu) rather than index arithmetic, so that an
indexing mistake in the oracle cannot be mirrored here.
"""

import numpy as np
import torch
import torch.nn.functional as F


def _t(a):
    return torch.from_numpy(np.asarray(a)).to(torch.float64)


def relative_position_index(window):
    coords = torch.stack(torch.meshgrid(torch.arange(window), torch.arange(window),
                                        indexing="ij")).flatten(1)
    rel = (coords[:, :, None] - coords[:, None, :]).permute(1, 2, 0).contiguous()
    rel[:, :, 0] += window - 1
    rel[:, :, 1] += window - 1
    rel[:, :, 0] *= 2 * window - 1
    return rel.sum(-1)


def shifted_window_msa(query, qkv_w, qkv_b, rel_bias, rel_index, proj_w, proj_b,
                       heads, window, shift):
    """[B,H,W,C] -> [B,H,W,C]; float64 throughout."""
    x = _t(query)
    b, h, w, c = x.shape
    pad_b = (window - h % window) % window
    pad_r = (window - w % window) % window
    x = F.pad(x, (0, 0, 0, pad_r, 0, pad_b))
    hp, wp = x.shape[1:3]
    mask = None
    if shift:
        x = torch.roll(x, shifts=(-shift, -shift), dims=(1, 2))
        img = torch.zeros(1, hp, wp, 1, dtype=torch.float64)
        label = 0
        for hs in (slice(0, -window), slice(-window, -shift), slice(-shift, None)):
            for ws in (slice(0, -window), slice(-window, -shift), slice(-shift, None)):
                img[:, hs, ws, :] = label
                label += 1
        mw = img.view(1, hp // window, window, wp // window, window, 1).permute(
            0, 1, 3, 2, 4, 5).reshape(-1, window * window)
        mask = mw.unsqueeze(1) - mw.unsqueeze(2)
        mask = mask.masked_fill(mask != 0, -100.0).masked_fill(mask == 0, 0.0)
    win = x.view(b, hp // window, window, wp // window, window, c).permute(
        0, 1, 3, 2, 4, 5).reshape(-1, window * window, c)
    nw, t, _ = win.shape
    qkv = F.linear(win, _t(qkv_w), _t(qkv_b)).reshape(nw, t, 3, heads, c // heads).permute(
        2, 0, 3, 1, 4)
    q, k, v = qkv[0], qkv[1], qkv[2]
    attn = (q * (c // heads) ** -0.5) @ k.transpose(-2, -1)
    bias = _t(rel_bias)[torch.as_tensor(np.asarray(rel_index)).reshape(-1)].view(t, t, heads)
    attn = attn + bias.permute(2, 0, 1).unsqueeze(0)
    if mask is not None:
        nwin = mask.shape[0]
        attn = attn.view(nw // nwin, nwin, heads, t, t) + mask.unsqueeze(1).unsqueeze(0)
        attn = attn.view(nw, heads, t, t)
    attn = attn.softmax(-1)
    y = (attn @ v).transpose(1, 2).reshape(nw, t, c)
    y = F.linear(y, _t(proj_w), _t(proj_b))
    y = y.view(b, hp // window, wp // window, window, window, c).permute(
        0, 1, 3, 2, 4, 5).reshape(b, hp, wp, c)
    if shift:
        y = torch.roll(y, shifts=(shift, shift), dims=(1, 2))
    return y[:, :h, :w].contiguous().numpy()


def patch_merge_unfold(x_bhwc):
    """nn.Unfold(2, stride 2) rows of a [B,H,W,C] map, zero padded to even."""
    x = _t(x_bhwc)
    b, h, w, c = x.shape
    x = F.pad(x, (0, 0, 0, w % 2, 0, h % 2))
    cols = F.unfold(x.permute(0, 3, 1, 2), kernel_size=2, stride=2)  # [B, C*4, L]
    return cols.transpose(1, 2).numpy()  # [B, L, 4C], element c*4 + ky*2 + kx


def bilinear_up(x_nchw, out_hw):
    return F.interpolate(_t(x_nchw), size=out_hw, mode="bilinear",
                         align_corners=False).numpy()


def layer_norm(x, g, b, eps=1e-5):
    x = _t(x)
    return F.layer_norm(x, (x.shape[-1],), _t(g), _t(b), eps).numpy()


def gelu(x):
    return F.gelu(_t(x), approximate="none").numpy()


# ---------------------------------------------------------------- modules
def _bn(x, p, prefix, eps=1e-5):
    return F.batch_norm(x, _t(p[prefix + ".running_mean"]), _t(p[prefix + ".running_var"]),
                        _t(p[prefix + ".weight"]), _t(p[prefix + ".bias"]), training=False,
                        eps=eps)


def _offset_ratio(x, sink):
    """Median over rows of |row mean| / row std of a LayerNorm input."""
    if sink is not None:
        mu = x.mean(-1)
        sd = x.std(-1, unbiased=False)
        sink.append(float((mu.abs() / sd).median()))


def swin_backbone(p, images, ln_offsets=None):
    """Swin-T (mmdet SwinTransformer, out_indices 1..3) in float64.

    ``p`` maps tensor names to arrays (the synthetic checkpoint).  With
    ``ln_offsets`` a list, the median |mean| / std of the rows entering each
    LayerNorm of stages 1-3 (norm1, norm2, the stage-output norm) is appended
    to it."""
    pre = "image_backbone."
    x = F.conv2d(_t(images), _t(p[pre + "patch_embed.projection.weight"]),
                 _t(p[pre + "patch_embed.projection.bias"]), stride=4)
    b, c, h, w = x.shape
    x = x.permute(0, 2, 3, 1)
    x = F.layer_norm(x, (c,), _t(p[pre + "patch_embed.norm.weight"]),
                     _t(p[pre + "patch_embed.norm.bias"]), 1e-5)
    outs = []
    for s, (c, heads, depth) in enumerate(zip((96, 192, 384, 768), (3, 6, 12, 24),
                                              (2, 2, 6, 2))):
        for k in range(depth):
            q = f"{pre}stages.{s}.blocks.{k}."
            _offset_ratio(x, ln_offsets if s > 0 else None)
            y = F.layer_norm(x, (c,), _t(p[q + "norm1.weight"]), _t(p[q + "norm1.bias"]), 1e-5)
            y = torch.from_numpy(shifted_window_msa(
                y.numpy(), p[q + "attn.w_msa.qkv.weight"], p[q + "attn.w_msa.qkv.bias"],
                p[q + "attn.w_msa.relative_position_bias_table"],
                p[q + "attn.w_msa.relative_position_index"], p[q + "attn.w_msa.proj.weight"],
                p[q + "attn.w_msa.proj.bias"], heads, 7, 3 if k % 2 else 0))
            x = x + y
            _offset_ratio(x, ln_offsets if s > 0 else None)
            y = F.layer_norm(x, (c,), _t(p[q + "norm2.weight"]), _t(p[q + "norm2.bias"]), 1e-5)
            y = F.gelu(F.linear(y, _t(p[q + "ffn.layers.0.0.weight"]),
                                _t(p[q + "ffn.layers.0.0.bias"])))
            x = x + F.linear(y, _t(p[q + "ffn.layers.1.weight"]), _t(p[q + "ffn.layers.1.bias"]))
        if s > 0:
            _offset_ratio(x, ln_offsets)
            o = F.layer_norm(x, (c,), _t(p[f"{pre}norm{s}.weight"]), _t(p[f"{pre}norm{s}.bias"]),
                             1e-5)
            outs.append(o.permute(0, 3, 1, 2).contiguous().numpy())
        if s < 3:
            q = f"{pre}stages.{s}.downsample."
            bsz, hh, ww, _ = x.shape
            cols = torch.from_numpy(patch_merge_unfold(x.numpy()))
            cols = F.layer_norm(cols, (4 * c,), _t(p[q + "norm.weight"]), _t(p[q + "norm.bias"]),
                                1e-5)
            x = F.linear(cols, _t(p[q + "reduction.weight"])).view(
                bsz, (hh + 1) // 2, (ww + 1) // 2, 2 * c)
    return outs


def _conv_bn_relu(x, p, w, b, bn, stride=1, pad=0, relu=True):
    y = F.conv2d(x, _t(p[w]), None if b is None else _t(p[b]), stride=stride, padding=pad)
    if bn:
        y = _bn(y, p, bn)
    return F.relu(y) if relu else y


def image_fpn(p, s0, s1, s2):
    """GeneralizedLSSFPN (2 levels, concat + 1x1 + 3x3, BN + ReLU)."""
    x0, x1, x2 = _t(s0), _t(s1), _t(s2)
    up = F.interpolate(x2, size=x1.shape[2:], mode="bilinear", align_corners=False)
    t = _conv_bn_relu(torch.cat([x1, up], 1), p, "neck.lateral_convs.1.conv.weight", None,
                      "neck.lateral_convs.1.bn")
    o1 = _conv_bn_relu(t, p, "neck.fpn_convs.1.conv.weight", None, "neck.fpn_convs.1.bn", pad=1)
    up = F.interpolate(o1, size=x0.shape[2:], mode="bilinear", align_corners=False)
    t = _conv_bn_relu(torch.cat([x0, up], 1), p, "neck.lateral_convs.0.conv.weight", None,
                      "neck.lateral_convs.0.bn")
    o0 = _conv_bn_relu(t, p, "neck.fpn_convs.0.conv.weight", None, "neck.fpn_convs.0.bn", pad=1)
    return o0.numpy(), o1.numpy()


def depth_head(p, features, depth):
    """DepthLSS: dtransform on dense depth, concat with features, depthnet."""
    v = "vtransform."
    d = _conv_bn_relu(_t(depth), p, v + "dtransform.0.weight", v + "dtransform.0.bias",
                      v + "dtransform.1")
    d = _conv_bn_relu(d, p, v + "dtransform.3.weight", v + "dtransform.3.bias",
                      v + "dtransform.4", stride=4, pad=2)
    d = _conv_bn_relu(d, p, v + "dtransform.6.weight", v + "dtransform.6.bias",
                      v + "dtransform.7", stride=2, pad=2)
    x = torch.cat([d, _t(features)], 1)
    x = _conv_bn_relu(x, p, v + "depthnet.0.weight", v + "depthnet.0.bias", v + "depthnet.1",
                      pad=1)
    x = _conv_bn_relu(x, p, v + "depthnet.3.weight", v + "depthnet.3.bias", v + "depthnet.4",
                      pad=1)
    x = F.conv2d(x, _t(p[v + "depthnet.6.weight"]), _t(p[v + "depthnet.6.bias"]))
    return x[:, :118].numpy(), x[:, 118:].numpy()


def lss_downsample(p, bev):
    v = "vtransform.downsample."
    x = _conv_bn_relu(_t(bev), p, v + "0.weight", None, v + "1", pad=1)
    x = _conv_bn_relu(x, p, v + "3.weight", None, v + "4", stride=2, pad=1)
    x = _conv_bn_relu(x, p, v + "6.weight", None, v + "7", pad=1)
    return x.transpose(2, 3).contiguous().numpy()


def bev_stage(p, x):
    """Fuser + SECOND backbone / deblocks + TransFusion shared conv and heatmap
    head (BatchNorm epsilon 1e-3) in float64: (spatial, shared, heatmap)."""
    def cbr(y, w, bn, stride=1, pad=1, bias=None, relu=True):
        y = F.conv2d(y, _t(p[w]), None if bias is None else _t(p[bias]), stride=stride,
                     padding=pad)
        if bn:
            y = _bn(y, p, bn, eps=1e-3)
        return F.relu(y) if relu else y

    y = cbr(_t(x), "fuser.conv.0.weight", "fuser.conv.1")
    for l in range(6):
        y = cbr(y, f"backbone_2d.blocks.0.{3 * l + 1}.weight", f"backbone_2d.blocks.0.{3 * l + 2}")
    up0 = cbr(y, "backbone_2d.deblocks.0.0.weight", "backbone_2d.deblocks.0.1", pad=0)
    for l in range(6):
        y = cbr(y, f"backbone_2d.blocks.1.{3 * l + 1}.weight", f"backbone_2d.blocks.1.{3 * l + 2}",
                stride=1 if l else 2)
    up1 = F.relu(_bn(F.conv_transpose2d(y, _t(p["backbone_2d.deblocks.1.0.weight"]), stride=2), p,
                     "backbone_2d.deblocks.1.1", eps=1e-3))
    spatial = torch.cat([up0, up1], 1)
    shared = cbr(spatial, "dense_head.shared_conv.weight", None,
                 bias="dense_head.shared_conv.bias", relu=False)
    mid = cbr(shared, "dense_head.heatmap_head.0.conv.weight", "dense_head.heatmap_head.0.bn")
    heat = cbr(mid, "dense_head.heatmap_head.1.weight", None,
               bias="dense_head.heatmap_head.1.bias", relu=False)
    return spatial.numpy(), shared.numpy(), heat.numpy()


def transfusion(p, shared, heatmap, proposals):
    """TransFusion head (mmdet3d TransFusionHead with one decoder layer) in
    float64: heatmap NMS by F.max_pool2d (interior 3x3 maxima; classes 8 and 9
    exempt; borders suppressed), top-k by a stable descending sort, query =
    features + class encoding, position embeddings, self and cross
    nn.MultiheadAttention through F.multi_head_attention_forward, FFN, three
    LayerNorms and the six prediction heads.  Returns the raw-output dict of
    oracle.Oracle.transfusion."""
    sh, hm = _t(shared)[0], torch.sigmoid(_t(heatmap))
    c, h, w = sh.shape
    keys = h * w
    local = torch.zeros_like(hm)
    if h > 2 and w > 2:
        local[:, :, 1:-1, 1:-1] = F.max_pool2d(hm, 3, 1, 0)
    local[:, 8], local[:, 9] = hm[:, 8], hm[:, 9]
    hm = hm * (hm == local)
    flat = hm[0].reshape(-1)
    order = torch.sort(flat, descending=True, stable=True).indices[:proposals]
    labels, index = order // keys, order % keys
    feat = sh.reshape(c, keys)
    query = feat[:, index] + _t(p["dense_head.class_encoding.weight"])[:, :, 0][:, labels] + \
        _t(p["dense_head.class_encoding.bias"])[:, None]
    query = query.T  # [P, C]

    def posembed(base, cells):
        x = (cells % w).to(torch.float64) + 0.5
        y = torch.div(cells, w, rounding_mode="floor").to(torch.float64) + 0.5
        q = f"dense_head.decoder.{base}.position_embedding_head."
        z = F.conv1d(torch.stack([x, y])[None], _t(p[q + "0.weight"]), _t(p[q + "0.bias"]))
        z = F.relu(_bn(z, p, q + "1"))
        return F.conv1d(z, _t(p[q + "3.weight"]), _t(p[q + "3.bias"]))[0].T

    query_pos = posembed("self_posembed", index)
    key_value = posembed("cross_posembed", torch.arange(keys)) + feat.T

    def mha(name, q, kv):
        pre = f"dense_head.decoder.{name}."
        out, _ = F.multi_head_attention_forward(
            q[:, None], kv[:, None], kv[:, None], 128, 8, _t(p[pre + "in_proj_weight"]),
            _t(p[pre + "in_proj_bias"]), None, None, False, 0.0,
            _t(p[pre + "out_proj.weight"]), _t(p[pre + "out_proj.bias"]), training=False,
            need_weights=False)
        return out[:, 0]

    def norm(x, i):
        pre = f"dense_head.decoder.norm{i}."
        return F.layer_norm(x, (128,), _t(p[pre + "weight"]), _t(p[pre + "bias"]), 1e-5)

    t = query + query_pos
    query = norm(query + mha("self_attn", t, t), 1)
    query = norm(query + mha("multihead_attn", query + query_pos, key_value), 2)
    d = "dense_head.decoder."
    ffn = F.linear(F.relu(F.linear(query, _t(p[d + "linear1.weight"]), _t(p[d + "linear1.bias"]))),
                   _t(p[d + "linear2.weight"]), _t(p[d + "linear2.bias"]))
    query = norm(query + ffn, 3)
    out = {}
    for key, head in (("center", "center"), ("height", "height"), ("dimension_log", "dim"),
                      ("rotation", "rot"), ("velocity", "vel"), ("heatmap_logits", "heatmap")):
        q = f"dense_head.prediction_head.{head}."
        z = F.conv1d(query.T[None], _t(p[q + "0.0.weight"]))
        z = F.relu(_bn(z, p, q + "0.1"))
        out[key] = F.conv1d(z, _t(p[q + "1.weight"]), _t(p[q + "1.bias"])).numpy()
    out["center"][0, 0] += (index % w).numpy() + 0.5
    out["center"][0, 1] += torch.div(index, w, rounding_mode="floor").numpy() + 0.5
    out["query_scores"] = hm[0].reshape(10, keys)[:, index][None].numpy()
    out["labels"] = labels[None].numpy()
    out["indices"] = index[None].numpy()
    return out
