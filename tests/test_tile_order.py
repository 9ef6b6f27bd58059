"""The workgroup -> tile maps of the GEMM cores (hip_common.h: xcd_swizzle and
the XCD-blocked order of the weight-heavy layers) are permutations of the tile
grid, checked on the host: a map that dropped or repeated a tile would leave
part of an output unwritten.  Compiles tests/tile_order_check.hip with hipcc
(host code only; nothing runs on a GPU)."""

import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def test_tile_maps_are_permutations(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not pathlib.Path(hipcc).exists():
        pytest.skip("hipcc not available")
    exe = tmp_path / "tile_order_check"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O1", "-std=c++17",
                    f"-I{ROOT / 'bevfusion.c_amd' / 'csrc'}", f"-I{ROOT / 'include'}",
                    str(ROOT / "tests" / "tile_order_check.hip"), "-o", str(exe)],
                   check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout + out.stderr
