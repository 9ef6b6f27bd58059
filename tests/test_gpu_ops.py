"""Parity of the stateless operators bf_cuda_gemm_f32 / bf_cuda_conv2d_f32.

Cases follow the reference's own GPU operator test (tests/test_cuda_ops.cu):
the 19x23->17 ReLU GEMM, a strided conv, a 5x5/s4 conv with Inf/NaN injected,
a 2x2/s2 transposed conv and a 1 048 561-row grid (65 536 row tiles), all with
its pattern() fill, plus BASELINE.json config 1 (11264x96 -> 288).

Two references per case:
  * the fp32 CPU oracle / float64 restatement of the operator, held to the
    north-star bf16 tolerance (tests/util.py);
  * the same float64 sum over bf16-rounded operands, held to 1e-5 relative:
    it isolates the kernel's indexing from bf16 input rounding, so a wrong
    tap, row or channel cannot hide inside the bf16 tolerance.
"""

import numpy as np
import pytest

import convref
from util import assert_close, bf16_round, pattern

pytestmark = pytest.mark.gpu


def _t(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(device)


def _tight(actual, expected, name, rtol=1e-5):
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    fin = np.isfinite(e)
    scale = np.sqrt(np.mean(e[fin] ** 2)) + 1e-30
    err = np.max(np.abs(a[fin] - e[fin])) / scale
    assert err <= rtol, f"{name}: bf16-operand residual {err:.3e} > {rtol:.1e}"


def run_conv(device, fields, inject_special=False):
    import bfhip
    d = bfhip.ConvDesc(*fields)
    n_in = d.batches * d.input_channels * d.input_height * d.input_width
    n_w = d.input_channels * d.output_channels * d.kernel_height * d.kernel_width
    x = pattern(np.arange(n_in)).reshape(d.batches, d.input_channels, d.input_height,
                                         d.input_width)
    if d.transpose:
        w = (pattern(np.arange(n_w) + 11) * np.float32(0.1)).reshape(
            d.input_channels, d.output_channels, d.kernel_height, d.kernel_width)
    else:
        w = (pattern(np.arange(n_w) + 11) * np.float32(0.1)).reshape(
            d.output_channels, d.input_channels, d.kernel_height, d.kernel_width)
    b = pattern(np.arange(d.output_channels) + 29) * np.float32(0.2)
    if inject_special:
        x.reshape(-1)[0] = np.inf
        w.reshape(-1)[0] = 0.0
        x.reshape(-1)[-1] = np.nan
    import torch
    out = torch.empty((d.batches, d.output_channels, d.output_height, d.output_width),
                      device=device)
    xt, wt, bt = _t(x, device), _t(w, device), _t(b, device)
    ok, msg = bfhip.conv2d_raw(d, xt.data_ptr(), wt.data_ptr(), bt.data_ptr(), out.data_ptr())
    assert ok, msg
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    return d, x, w, b, got


CONV_CASES = {
    # fields: batches, Ci, Co, IH, IW, KH, KW, SH, SW, PH, PW, OH, OW, transpose, relu
    "stride": ((2, 3, 5, 6, 7, 3, 3, 2, 2, 1, 1, 3, 4, 0, 1), False),
    "wide_inf_nan": ((1, 2, 3, 9, 10, 5, 5, 4, 4, 2, 2, 3, 3, 0, 0), True),
    "transpose": ((1, 3, 5, 4, 6, 2, 2, 2, 2, 0, 0, 8, 12, 1, 1), False),
    "large_grid": ((1, 1, 1, 1, 1048561, 1, 1, 1, 1, 0, 0, 1, 1048561, 0, 0), False),
    "k3_c64_relu": ((2, 64, 96, 13, 17, 3, 3, 1, 1, 1, 1, 13, 17, 0, 1), False),
    "k5_s2_odd": ((1, 7, 33, 21, 19, 5, 5, 2, 2, 2, 2, 11, 10, 0, 0), False),
}


@pytest.mark.parametrize("case", sorted(CONV_CASES))
def test_conv_reference_cases(device, case):
    fields, special = CONV_CASES[case]
    d, x, w, b, got = run_conv(device, fields, special)
    expected = convref.conv_abi(d, x, w, b)
    assert_close(got, expected, case)
    _tight(got, convref.conv_abi(d, x, w, b, round_inputs=bf16_round), case)


def test_conv_matches_oracle(device):
    """Strided conv with bias against the CPU oracle (oracle port, OpenMP)."""
    import oracle
    import bfhip
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 16, 20, 24)).astype(np.float32)
    w = (rng.standard_normal((40, 16, 3, 3)) / 12).astype(np.float32)
    b = rng.standard_normal(40).astype(np.float32)
    ref = oracle.Oracle("port").conv2d(x, w, b, stride=(2, 2), pad=(1, 1))
    got = bfhip.conv2d_f32(_t(x, device), _t(w, device), _t(b, device), stride=(2, 2),
                           padding=(1, 1)).cpu().numpy()
    assert_close(got, ref, "conv vs oracle")


def test_conv_transpose_matches_oracle(device):
    import oracle
    import bfhip
    rng = np.random.default_rng(4)
    x = rng.standard_normal((1, 6, 5, 7)).astype(np.float32)
    w = (rng.standard_normal((6, 10, 2, 2)) / 3).astype(np.float32)  # IOHW
    b = rng.standard_normal(10).astype(np.float32)
    ref = oracle.Oracle("port").conv_transpose2d(x, w, b, stride=(2, 2))
    got = bfhip.conv2d_f32(_t(x, device), _t(w, device), _t(b, device), stride=(2, 2),
                           transpose=True).cpu().numpy()
    assert_close(got, ref, "transposed conv vs oracle")


def test_gemm_reference_fixture(device):
    """test_cuda_ops.cu:118-153: 19x23 -> 17, bias, ReLU, pattern() fill."""
    import bfhip
    rows, k, n = 19, 23, 17
    a = pattern(np.arange(rows * k)).reshape(rows, k) * np.float32(0.2)
    w = pattern(np.arange(n * k) + 7).reshape(n, k) * np.float32(0.1)
    b = pattern(np.arange(n) + 3)
    got = bfhip.gemm_f32(_t(a, device), _t(w, device), _t(b, device), relu=True).cpu().numpy()
    assert_close(got, convref.gemm_abi(a, w, b, True), "gemm 19x23x17")
    _tight(got, convref.gemm_abi(a, w, b, True, round_inputs=bf16_round), "gemm 19x23x17")


def test_gemm_config1_matches_oracle(device):
    """X[11264x96] W[288x96] + bias, ~N(0,1)/sqrt(96), seed 0."""
    import oracle
    import bfhip
    from bfhip import bfw
    x = bfw.randn(0, "config1.x", (11264, 96), 1 / np.sqrt(96))
    w = bfw.randn(0, "config1.w", (288, 96), 1 / np.sqrt(96))
    b = bfw.randn(0, "config1.b", (288,), 1 / np.sqrt(96))
    ref = oracle.Oracle("port").linear(x, w, b)
    got = bfhip.gemm_f32(_t(x, device), _t(w, device), _t(b, device)).cpu().numpy()
    assert_close(got, ref, "config1 linear")
    _tight(got, convref.gemm_abi(x, w, b, False, round_inputs=bf16_round), "config1 linear")


@pytest.mark.parametrize("shape", [(1, 1, 1), (7, 5, 4), (300, 96, 96), (129, 130, 131),
                                   (1000, 384, 1536), (64, 3072, 768), (513, 8, 33),
                                   (200, 96, 145), (77, 31, 250), (33, 64, 288)])
def test_gemm_shapes(device, shape):
    import bfhip
    m, k, n = shape
    rng = np.random.default_rng(m * 7 + k * 3 + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    got = bfhip.gemm_f32(_t(x, device), _t(w, device), _t(b, device)).cpu().numpy()
    assert_close(got, convref.gemm_abi(x, w, b, False), f"gemm {shape}")
    _tight(got, convref.gemm_abi(x, w, b, False, round_inputs=bf16_round), f"gemm {shape}")


def test_gemm_unaligned_operands(device):
    """Row pitch not a multiple of 4 floats and offset base pointers (scalar path)."""
    import bfhip
    import torch
    rng = np.random.default_rng(9)
    x = rng.standard_normal((50, 31)).astype(np.float32)
    w = rng.standard_normal((20, 31)).astype(np.float32)
    xt = torch.zeros(50 * 31 + 1, device=device)
    xt[1:] = _t(x, device).reshape(-1)
    xv = xt[1:].view(50, 31)
    got = bfhip.gemm_f32(xv, _t(w, device)).cpu().numpy()
    _tight(got, convref.gemm_abi(x, w, None, False, round_inputs=bf16_round), "unaligned")


def test_repeat_is_bit_exact(device):
    """Determinism gate (reference test_cuda_camera_full.cu:69-72): no atomics."""
    import bfhip
    rng = np.random.default_rng(5)
    x = _t(rng.standard_normal((4096, 384)), device)
    w = _t(rng.standard_normal((1152, 384)) / 20, device)
    a = bfhip.gemm_f32(x, w).cpu().numpy()
    b = bfhip.gemm_f32(x, w).cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# (rows, in, out, relu, bias, inject Inf/NaN): shapes the short-reduction
# panel kernel takes (K <= 128, K % 4 == 0, 144 < N <= 288, N % 4 == 0):
# ragged row panels, N not a multiple of 16, K not a multiple of 8 or 32,
# one to four 32-deep k-steps, ReLU, no bias, and Inf/NaN operands.
PANEL_CASES = [(1001, 100, 148, True, True, False), (64, 4, 160, False, False, False),
               (5, 128, 200, False, True, False), (130, 32, 288, True, True, True),
               (11264, 96, 288, False, True, False), (65, 60, 252, False, True, False)]


@pytest.mark.parametrize("case", PANEL_CASES)
def test_gemm_panel_equals_tiled_core(device, case):
    """The panel kernel (aligned operands) against the tiled core, reached by
    handing the library an output that is not 16-byte aligned: same bf16
    operand rounding, same 32-deep k order and bias after the accumulation,
    so the two must agree bit for bit; and both within 1e-5 of the float64
    sum over bf16-rounded operands."""
    import bfhip
    import torch
    m, k, n, relu, with_bias, special = case
    print(f"[case] panel gemm {m}x{k}->{n} relu={relu} bias={with_bias} special={special}",
          flush=True)
    rng = np.random.default_rng(m + 3 * k + 7 * n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32) if with_bias else None
    if special:
        x[0, 0] = np.inf
        x[-1, -1] = np.nan
    xt, wt = _t(x, device), _t(w, device)
    bt = _t(b, device) if with_bias else None
    panel = bfhip.gemm_f32(xt, wt, bt, relu=relu)
    buf = torch.empty(m * n + 1, device=device)
    tiled_out = buf[1:].view(m, n)
    bfhip.gemm_f32(xt, wt, bt, relu=relu, out=tiled_out)
    torch.cuda.synchronize()
    a, t = panel.cpu().numpy(), tiled_out.cpu().numpy()
    assert np.array_equal(a.view(np.uint32), t.view(np.uint32)), "panel and tiled core differ"
    want = convref.gemm_abi(x, w, b, relu, round_inputs=bf16_round)
    if special:
        assert np.array_equal(np.isnan(a), np.isnan(want)) and np.array_equal(np.isinf(a), np.isinf(want))
    _tight(a, want, f"panel gemm {case}")
