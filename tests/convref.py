"""Independent float64 references for the stateless operator ABI.

These restate the operator semantics of reference include/bf_cuda_ops.h (the
host references of tests/test_cuda_ops.cu:22-71,118-131) with numpy, tap by
tap, so they share no code with either the oracle or the HIP library.
"""

import numpy as np


def conv_abi(desc, x, w, b, relu=None, round_inputs=None):
    """Convolution per bf_cuda_conv2d_desc fields; x NCHW, w OIHW or IOHW."""
    d = desc
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.float32)
    if round_inputs is not None:
        x, w = round_inputs(x), round_inputs(w)
    x = x.astype(np.float64)
    w = w.astype(np.float64)
    N, Ci, IH, IW = d.batches, d.input_channels, d.input_height, d.input_width
    Co, KH, KW = d.output_channels, d.kernel_height, d.kernel_width
    OH, OW = d.output_height, d.output_width
    out = np.zeros((N, Co, OH, OW), np.float64)
    oy = np.arange(OH)[:, None]
    ox = np.arange(OW)[None, :]
    with np.errstate(invalid="ignore", over="ignore"):
        for ky in range(KH):
            for kx in range(KW):
                if not d.transpose:
                    iy = oy * d.stride_height - d.padding_height + ky
                    ix = ox * d.stride_width - d.padding_width + kx
                    tap = np.ones((OH, OW), bool)
                else:
                    sy = oy + d.padding_height - ky
                    sx = ox + d.padding_width - kx
                    tap = (sy >= 0) & (sx >= 0) & (sy % d.stride_height == 0) & \
                          (sx % d.stride_width == 0)
                    iy = np.where(tap, sy // d.stride_height, -1)
                    ix = np.where(tap, sx // d.stride_width, -1)
                iy = np.broadcast_to(iy, (OH, OW))
                ix = np.broadcast_to(ix, (OH, OW))
                valid = tap & (iy >= 0) & (iy < IH) & (ix >= 0) & (ix < IW)
                if not valid.any():
                    continue
                g = np.zeros((N, Ci, OH, OW), np.float64)
                g[:, :, valid] = x[:, :, iy[valid], ix[valid]]
                wk = w[:, :, ky, kx] if not d.transpose else w[:, :, ky, kx].T  # [Co, Ci]
                # Only valid taps contribute (so 0 * Inf padding never appears).
                contrib = np.einsum("oc,nchw->nohw", wk, g)
                out += np.where(valid[None, None], contrib, 0.0)
    if b is not None:
        out += np.asarray(b, np.float64)[None, :, None, None]
    r = d.relu if relu is None else relu
    if r:
        out = np.where(out < 0, 0.0, out)
    return out


def gemm_abi(x, w, b, relu, round_inputs=None):
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.float32)
    if round_inputs is not None:
        x, w = round_inputs(x), round_inputs(w)
    y = x.astype(np.float64) @ w.astype(np.float64).T
    if b is not None:
        y += np.asarray(b, np.float64)[None]
    return np.maximum(y, 0.0) if relu else y
