"""Window attention without allocation (bfhip_debug_window_attention_noalloc,
include/bfhip_debug.h) against the allocating probe it mirrors
(bfhip_debug_window_attention): both build the same score terms with the same
kernel and run the same attention kernel, so their outputs must agree bit for
bit.  The no-allocation entry point is called twice in a row, the second time
on a smaller problem (fewer tokens, fewer heads, another window shift), so the
second call runs on a static term array that still holds the first call's
larger terms.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (batches, height, width, heads, shift): a larger call, then a smaller one.
CASES = [
    ((2, 56, 112, 6, 3), (1, 14, 21, 3, 0)),
    ((6, 16, 44, 24, 3), (2, 9, 12, 12, 3)),
    ((1, 8, 22, 32, 0), (1, 7, 7, 2, 3)),
]


def _inputs(seed, shape, device):
    import torch
    b, h, w, heads, _ = shape
    c, tokens = 32 * heads, b * h * w
    r = np.random.default_rng(seed)
    qkv = torch.from_numpy((0.5 * r.standard_normal((tokens, 3 * c))).astype(np.float32))
    qkv_bias = torch.from_numpy((0.1 * r.standard_normal(3 * c)).astype(np.float32))
    bias_mat = torch.from_numpy((0.5 * r.standard_normal((heads, 49, 49))).astype(np.float32))
    return (qkv.to(device).to(torch.float16), qkv_bias.to(device), bias_mat.to(device))


@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_window_attention_matches_allocating_probe(device, first, second):
    import bfhip
    import torch
    shapes = (first, second)
    inputs = [_inputs(11 + i, s, device) for i, s in enumerate(shapes)]
    want = []
    for shape, args in zip(shapes, inputs):
        b, h, w, heads, shift = shape
        print(f"[case] allocating probe b={b} h={h} w={w} heads={heads} shift={shift}", flush=True)
        want.append(bfhip.window_attention(*args, b, h, w, heads, shift))
    torch.cuda.synchronize()
    got = []
    for shape, args in zip(shapes, inputs):   # two no-allocation calls in a row
        b, h, w, heads, shift = shape
        print(f"[case] no-allocation b={b} h={h} w={w} heads={heads} shift={shift}", flush=True)
        got.append(bfhip.window_attention(*args, b, h, w, heads, shift, noalloc=True))
    torch.cuda.synchronize()
    for shape, g, e in zip(shapes, got, want):
        assert torch.isfinite(e.float()).all() and e.float().abs().max() > 0, shape
        assert torch.equal(g, e), f"{shape}: no-allocation output differs from the probe's"


def test_noalloc_window_attention_rejects_too_many_heads(device):
    import bfhip
    import torch
    shape = (1, 7, 7, 33, 0)
    args = _inputs(5, shape, device)
    with pytest.raises(bfhip.BfHipError, match="at most 32 heads"):
        bfhip.window_attention(*args, 1, 7, 7, 33, 0, noalloc=True)
    torch.cuda.synchronize()


def test_noalloc_window_attention_under_graph_capture(device):
    """Two no-allocation calls captured in one HIP graph (torch.cuda.graph),
    the second on a smaller problem; every replay, with eager work and
    synchronisation between replays, must equal the allocating probe bit for
    bit.  The captured kernels write the score terms into the static array at
    replay time, so nothing is allocated inside or after the capture."""
    import bfhip
    import torch
    shapes = CASES[0]
    inputs = [_inputs(31 + i, s, device) for i, s in enumerate(shapes)]
    want = [bfhip.window_attention(*args, *s) for s, args in zip(shapes, inputs)]
    outs = [torch.zeros_like(w) for w in want]
    # One eager call first: resolves the device's array before the capture.
    bfhip.window_attention(*inputs[1], *shapes[1], out=outs[1], noalloc=True)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for s, args, o in zip(shapes, inputs, outs):
            bfhip.window_attention(*args, *s, out=o, noalloc=True)
    for rep in range(4):
        print(f"[case] graph replay {rep}", flush=True)
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for s, o, w in zip(shapes, outs, want):
            assert torch.equal(o, w), f"replay {rep} {s}: differs from the allocating probe"
        # eager work between replays (the same entry point on another problem)
        bfhip.window_attention(*inputs[0], *shapes[0], noalloc=True)
        torch.cuda.synchronize()
