"""The CPU frame runtime restated (oracle/src/runtime.c) against the
reference's own src/runtime.c compiled as-is (oracle/_ref), on a full
synthetic frame: six 256 x 704 images, 100k points over ten sweeps, a
complete random-init checkpoint.  The two chains agree bit for bit on every
detection (both OpenMP builds; each module is separately pinned on the scalar
path).  Skipped where the reference sources are absent.
"""

import numpy as np
import pytest

import oracle
from bfhip import bfw, frame_scene


def test_runtime_bit_exact_with_reference(tmp_path):
    if not oracle.available("ref"):
        pytest.skip("reference CPU sources are not present to build oracle/_ref")
    path = bfw.write_full_model(tmp_path / "full.bfw", seed=1)
    frame = frame_scene.frame(1, 100000, sweeps=10)
    a = oracle.detections_array(oracle.Oracle("port").runtime_infer(path, frame))
    b = oracle.detections_array(oracle.Oracle("ref").runtime_infer(path, frame))
    assert a.shape == b.shape and a.shape[0] > 0
    assert np.array_equal(a, b)
