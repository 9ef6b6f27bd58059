"""Shared test configuration.

Markers: ``gpu`` tests need an MI355X (gfx950) and call the HIP library
through its C ABI; everything else runs on the CPU.
"""

import os
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "bevfusion.c_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU; calls libbfhip.so")


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but no GPU is visible")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def tmp_models(tmp_path_factory):
    """Synthetic checkpoints written once per session."""
    from bfhip import bfw
    base = tmp_path_factory.mktemp("models")
    cache = {}

    def get(mode="fan_in", seed=1, gain=1.0, offset=0.0):
        key = (mode, seed, gain, offset)
        if key not in cache:
            cache[key] = bfw.write_camera_branch(base / f"cam_{mode}_{seed}_{gain}_{offset}.bfw",
                                                 seed=seed, mode=mode, gain=gain, offset=offset)
        return cache[key]
    return get
