"""Parity of the Swin-T context (bf_cuda_swin_*) against the CPU oracle.

Weights are the synthetic checkpoint with fan-in scaled weights (every
residual branch contributes O(1), so a wrong branch cannot hide under the
residual stream).  Shapes: the reference's compact test (1x32x48,
tests/test_cuda_swin.cu:19), a 2-camera map whose stage-0/1 grids need no
window padding, one production camera (256x704), and the full 6-camera
production context checked through batch invariance and repeat exactness.
"""

import numpy as np
import pytest

from util import assert_close

pytestmark = pytest.mark.gpu


def _run_swin(model_path, images, device):
    import bfhip
    import torch
    b, _, h, w = images.shape
    with bfhip.Model(model_path) as m:
        ctx = bfhip.Swin(m, b, h, w)
    x = torch.from_numpy(images).to(device)
    outs = ctx.forward(x)
    torch.cuda.synchronize()
    res = [o.cpu().numpy() for o in outs]
    ctx.close()
    return res


def _oracle_swin(model_path, images):
    import oracle
    o = oracle.Oracle("port")
    with o.open_model(model_path) as m:
        return o.swin_backbone(m, images)


@pytest.mark.parametrize("shape", [(1, 32, 48), (2, 56, 112), (1, 256, 704)])
def test_swin_matches_oracle(device, tmp_models, shape):
    from bfhip import bfw
    path = tmp_models("fan_in", 1)
    images = bfw.synthetic_images(7, *shape)
    got = _run_swin(path, images, device)
    ref = _oracle_swin(path, images)
    for i, (g, r) in enumerate(zip(got, ref)):
        assert g.shape == r.shape
        assert np.isfinite(g).all()
        assert_close(g, r, f"swin {shape} output{i}")


def test_swin_baseline_init_matches_oracle(device, tmp_models):
    """BASELINE.json weight init (N(0,0.02)) at one production camera."""
    from bfhip import bfw
    path = tmp_models("baseline", 0)
    images = bfw.synthetic_images(0, 1, 256, 704)
    got = _run_swin(path, images, device)
    ref = _oracle_swin(path, images)
    for i, (g, r) in enumerate(zip(got, ref)):
        assert_close(g, r, f"swin baseline output{i}")


def test_swin_production_batch_invariance_and_repeat(device, tmp_models):
    """6x3x256x704 production context: camera k of a 6-camera forward is
    bit-identical to the 1-camera forward of the same image (no cross-camera
    coupling, no atomics), and repeated forwards are bit-identical."""
    import bfhip
    import torch
    from bfhip import bfw
    path = tmp_models("fan_in", 1)
    images = bfw.synthetic_images(11, 6, 256, 704)
    with bfhip.Model(path) as m:
        six = bfhip.Swin(m, 6, 256, 704)
        one = bfhip.Swin(m, 1, 256, 704)
    x = torch.from_numpy(images).to(device)
    a = six.forward(x)
    b = six.forward(x)
    torch.cuda.synchronize()
    for oa, ob in zip(a, b):
        assert torch.equal(oa, ob), "repeat forward differs"
    for cam in (0, 3, 5):
        single = one.forward(x[cam:cam + 1].contiguous())
        torch.cuda.synchronize()
        for oa, os in zip(a, single):
            assert torch.equal(oa[cam:cam + 1], os), f"camera {cam} depends on batch"
    six.close()
    one.close()


def test_swin_unaligned_images_match_aligned(device, tmp_models):
    """Images that start 4 bytes past a 16-byte boundary (a valid fp32
    pointer for the C ABI) take the scalar patch gather instead of the float4
    one; both stage the same fp16 operands, so every output is bit-identical
    to the aligned forward."""
    import bfhip
    import torch
    from bfhip import bfw
    path = tmp_models("fan_in", 1)
    images = bfw.synthetic_images(5, 2, 32, 48)
    x = torch.from_numpy(images).to(device)
    buf = torch.empty(x.numel() + 1, device=device)
    buf[1:].copy_(x.reshape(-1))
    xu = buf[1:].view(x.shape)
    assert xu.data_ptr() % 16 == 4
    with bfhip.Model(path) as m:
        ctx = bfhip.Swin(m, 2, 32, 48)
    a = ctx.forward(x)
    b = ctx.forward(xu)
    torch.cuda.synchronize()
    for oa, ob in zip(a, b):
        assert torch.equal(oa, ob), "unaligned images change the result"
    ctx.close()


@pytest.mark.parametrize("offset", [10.0, 30.0])
def test_swin_offset_rows_match_oracle(device, tmp_models, offset):
    """Residual rows with a large common offset.  The attention-proj and fc2
    biases of every block carry +offset, so the rows entering the LayerNorms
    of stages 1-3 have |mean| up to 50x (offset 10) and 150x (offset 30)
    their spread (median over rows, measured with the float64 restatement and
    asserted here).  Those LayerNorms are folded into the linears that
    consume them: the fp16 copy of the residual stream carries the offset
    into the matrix product, the reason this case is tested on its own."""
    import torchref
    from bfhip import bfw
    path = tmp_models("fan_in", 1, 1.0, offset)
    images = bfw.synthetic_images(7, 1, 64, 96)
    ratios = []
    torchref.swin_backbone(dict(bfw.camera_branch_tensors(1, "fan_in", 1.0, offset)), images,
                           ratios)
    assert max(ratios) >= 4.5 * offset and sorted(ratios)[len(ratios) // 2] >= 2 * offset, ratios
    got = _run_swin(path, images, device)
    ref = _oracle_swin(path, images)
    for i, (g, r) in enumerate(zip(got, ref)):
        assert np.isfinite(g).all()
        rel = float(np.linalg.norm(g - r) / np.linalg.norm(r))
        mx = float(np.abs(g - r).max() / np.sqrt(np.mean(r * r)))
        print(f"offset {offset} output{i}: rel-L2 {rel:.3e}, max-abs {mx:.3e} x RMS", flush=True)
        assert_close(g, r, f"swin offset {offset} output{i}")


@pytest.mark.parametrize("shape", [(2, 56, 112), (6, 256, 704)])
def test_swin_fused_merge_out_norm_matches_forward(device, tmp_models, shape):
    """The forward runs the merges after stages 1 and 2 in one launch with
    that stage's output LayerNorm (merge_out_ln_kernel).  After a forward the
    context still holds stage 2's residual, row statistics and fp16 copy
    (stage 3's live elsewhere), so the profiling hook that runs the same
    fused launch for stage 2 (include/bfhip_profile.h,
    BFHIP_SWIN_MERGE_OUT_NORM) and the standalone stage-2 LayerNorm must both
    reproduce the forward's second output bit for bit; and stage 3's
    standalone LayerNorm, run before them, the third."""
    import bfhip
    import torch
    from bfhip import bfw
    b, h, w = shape
    print(f"[case] fused merge + output norm, {shape}", flush=True)
    path = tmp_models("fan_in", 1)
    images = bfw.synthetic_images(7, b, h, w)
    x = torch.from_numpy(images).to(device)
    with bfhip.Model(path) as m:
        ctx = bfhip.Swin(m, b, h, w)
    outs = ctx.forward(x)
    torch.cuda.synchronize()
    fused = torch.full_like(outs[1], float("nan"))
    alone = torch.full_like(outs[1], float("nan"))
    last = torch.full_like(outs[2], float("nan"))
    # Stage 3's norm first: the merge in the fused launch rewrites stage 3's
    # residual (with the merge output, before stage 3's blocks).
    ctx.profile_io("out_norm", 3, out=last)
    ctx.profile_io("merge_out_norm", 2, out=fused)
    ctx.profile_io("out_norm", 2, out=alone)
    torch.cuda.synchronize()
    assert torch.equal(fused, outs[1]), "fused launch's output norm differs from the forward's"
    assert torch.equal(alone, outs[1]), "standalone output norm differs from the fused one"
    assert torch.equal(last, outs[2])
    ctx.close()
