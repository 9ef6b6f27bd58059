"""Bit-exact device index maps of the Swin window path and of the implicit-GEMM
convolution, against oracle/index_maps.py (itself pinned on the CPU by
tests/test_index_maps.py).

* Window partition / cyclic shift / region labels: the device functions the
  attention kernel uses, read out through bfhip_debug_window_map.
* The attention kernel's gather and scatter: with q = k = 0 and a relative
  bias that is 0 on one key per query (a permutation) and -1000 elsewhere,
  softmax is exactly one-hot, so every output row must equal, bit for bit, the
  v row of the token the oracle's map puts at the permuted window position
  (v holds small integers, exact in fp16, the Swin operand format).
* Shifted-window mask: with a zero bias, each query averages exactly the keys
  of its own region (-100 elsewhere), which the oracle's labels predict; in
  unshifted blocks the padded keys (v = qkv bias) take part.
* im2col addressing of bf_cuda_conv2d_f32 (direct and transposed): with
  one-hot weights W[co][k] = (co == k) the output is the im2col matrix itself;
  inputs are 1 + base-256 digits of their flat index (exact in bf16), so each
  output decodes to the input element it was read from.
"""

import numpy as np
import pytest

from oracle import index_maps

pytestmark = pytest.mark.gpu

SHAPES = [(1, 7, 7, 0), (2, 9, 12, 3), (1, 3, 4, 3), (1, 8, 22, 3), (6, 64, 176, 3),
          (6, 32, 88, 0), (2, 16, 44, 3)]


@pytest.mark.parametrize("shape", SHAPES)
def test_window_map_bit_exact(device, shape):
    import bfhip
    import torch
    b, h, w, shift = shape
    token, label = bfhip.window_map(b, h, w, shift, device)
    torch.cuda.synchronize()
    et, el = index_maps.window_map(b, h, w, shift)
    np.testing.assert_array_equal(token.cpu().numpy(), et)
    np.testing.assert_array_equal(label.cpu().numpy(), el)


def _encode_tokens(tokens, heads):
    """v row of token id: dims 0-2 = 1 + base-256 digits, dim 3 = head + 1."""
    ids = np.arange(tokens, dtype=np.int64)
    v = np.zeros((tokens, heads, 32), np.float32)
    for d in range(3):
        v[:, :, d] = 1 + (ids[:, None] >> (8 * d)) % 256
    v[:, :, 3] = np.arange(1, heads + 1)[None, :]
    return v.reshape(tokens, heads * 32)


@pytest.mark.parametrize("shape", SHAPES)
def test_window_attention_gather_scatter_bit_exact(device, shape):
    import bfhip
    import torch
    b, h, w, shift = shape
    heads = 3 if h * w > 2000 else 2
    c, tokens = 32 * heads, b * h * w
    v = _encode_tokens(tokens, heads)
    qkv = np.zeros((tokens, 3 * c), np.float32)
    qkv[:, 2 * c:] = v
    perm = np.array([[(3 * i + 5 + hh) % 49 for i in range(49)] for hh in range(heads)])
    bias_mat = np.full((heads, 49, 49), -1000.0, np.float32)
    for hh in range(heads):
        bias_mat[hh, np.arange(49), perm[hh]] = 0.0
    qkv_bias = np.zeros(3 * c, np.float32)   # padded keys carry v = 0
    q = torch.from_numpy(qkv).to(device).to(torch.float16)
    out = bfhip.window_attention(q, torch.from_numpy(qkv_bias).to(device),
                                 torch.from_numpy(bias_mat).to(device), b, h, w, heads, shift)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(tokens, heads, 32)

    token, _ = index_maps.window_map(b, h, w, shift)
    token = token.reshape(-1, 49)
    expect = np.full((tokens, heads, 32), np.nan, np.float32)
    vv = v.reshape(tokens, heads, 32)
    for hh in range(heads):
        dst = token                              # [windows, 49] query token rows
        src = token[:, perm[hh]]                 # key token each query selects
        rows = dst >= 0
        sel = np.where(src >= 0, src, 0)
        vals = np.where((src >= 0)[..., None], vv[sel, hh], 0.0)
        expect[dst[rows], hh] = vals[rows]
    assert not np.isnan(expect).any(), "every token is some window's query exactly once"
    np.testing.assert_array_equal(got, expect)


@pytest.mark.parametrize("shape", [(2, 9, 12, 3), (1, 3, 4, 3), (1, 8, 22, 3), (2, 16, 44, 3),
                                   (2, 9, 12, 0), (1, 8, 22, 0)])
def test_window_attention_region_mask(device, shape):
    import bfhip
    import torch
    b, h, w, shift = shape
    heads, c, tokens = 2, 64, b * h * w
    r = np.random.default_rng(3)
    v = r.integers(1, 64, size=(tokens, c)).astype(np.float32)
    qkv = np.zeros((tokens, 3 * c), np.float32)
    qkv[:, 2 * c:] = v
    qkv_bias = np.zeros(3 * c, np.float32)
    qkv_bias[2 * c:] = r.integers(1, 64, size=c)      # v of zero-padded keys
    bias_mat = np.zeros((heads, 49, 49), np.float32)
    out = bfhip.window_attention(torch.from_numpy(qkv).to(device).to(torch.float16),
                                 torch.from_numpy(qkv_bias).to(device),
                                 torch.from_numpy(bias_mat).to(device), b, h, w, heads, shift)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()

    token, label = index_maps.window_map(b, h, w, shift)
    token, label = token.reshape(-1, 49), label.reshape(-1, 49)
    vals = np.where((token >= 0)[..., None], v[np.maximum(token, 0)], qkv_bias[2 * c:])
    expect = np.zeros((tokens, c))
    for wi in range(token.shape[0]):
        same = label[wi][:, None] == label[wi][None, :] if shift else np.ones((49, 49), bool)
        mean = (same.astype(np.float64) @ vals[wi]) / same.sum(1, keepdims=True)
        rows = token[wi] >= 0
        expect[token[wi][rows]] = mean[rows]
    err = np.abs(got - expect) / np.abs(expect)
    assert err.max() <= 2.0 ** -8, f"max relative error {err.max():.3e}"


CONV_CASES = {
    # batches, Ci, Co(=K), IH, IW, KH, KW, SH, SW, PH, PW, OH, OW, transpose
    "stride": (2, 3, 27, 6, 7, 3, 3, 2, 2, 1, 1, 3, 4, 0),
    "k5_s4": (1, 2, 50, 9, 10, 5, 5, 4, 4, 2, 2, 3, 3, 0),
    "transpose_2x2_s2": (1, 3, 12, 4, 6, 2, 2, 2, 2, 0, 0, 8, 12, 1),
    "transpose_3x3_s2_p1": (1, 4, 36, 5, 5, 3, 3, 2, 2, 1, 1, 9, 9, 1),
    "k5_s2_odd": (1, 7, 175, 21, 19, 5, 5, 2, 2, 2, 2, 11, 10, 0),
    "k3_c64": (2, 64, 576, 13, 17, 3, 3, 1, 1, 1, 1, 13, 17, 0),
    "1x1": (2, 40, 40, 8, 8, 1, 1, 1, 1, 0, 0, 8, 8, 0),
}


@pytest.mark.parametrize("case", sorted(CONV_CASES))
def test_conv_im2col_bit_exact(device, case):
    import bfhip
    import torch
    n, ci, k, ih, iw, kh, kw, sh, sw, ph, pw, oh, ow, tr = CONV_CASES[case]
    assert k == ci * kh * kw
    n_in = n * ci * ih * iw
    if tr:   # IOHW: W[ci][co][ky][kx] = (co == ci*KH*KW + ky*KW + kx)
        w = np.eye(k, dtype=np.float32).reshape(ci, kh, kw, k).transpose(0, 3, 1, 2)
    else:    # OIHW: W[co][k] = (co == k)
        w = np.eye(k, dtype=np.float32).reshape(k, ci, kh, kw)
    d = bfhip.ConvDesc(n, ci, k, ih, iw, kh, kw, sh, sw, ph, pw, oh, ow, tr, 0)
    wt = torch.from_numpy(np.ascontiguousarray(w)).to(device)
    digits = []
    for dgt in range(3):
        x = (1 + (np.arange(n_in) >> (8 * dgt)) % 256).astype(np.float32)
        xt = torch.from_numpy(x).to(device)
        out = torch.empty((n, k, oh, ow), device=device)
        ok, msg = bfhip.conv2d_raw(d, xt.data_ptr(), wt.data_ptr(), None, out.data_ptr())
        assert ok, msg
        torch.cuda.synchronize()
        digits.append(out.cpu().numpy().transpose(0, 2, 3, 1).reshape(n * oh * ow, k))
    zero = digits[0] == 0
    for dg in digits:
        assert np.array_equal(dg == 0, zero)
    got = sum((dg.astype(np.int64) - 1) << (8 * i) for i, dg in enumerate(digits))
    got[zero] = -1
    expect = index_maps.conv_im2col(n, ci, ih, iw, kh, kw, sh, sw, ph, pw, oh, ow, tr)
    np.testing.assert_array_equal(got, expect)
