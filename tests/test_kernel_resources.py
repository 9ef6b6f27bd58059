"""Register, scratch and LDS use of the library's kernels (CPU only), from the
compiler's kernel-resource-usage remarks that build() records in
bevfusion.c_amd/_build/kernel_resources.json.

Every kernel of the library runs without scratch memory and without
vector-register spills (SGPR spills go to VGPR lanes, not memory): a kernel
that uses scratch pays for it on every dispatch (a by-value struct kernel
argument read through a reference was once copied to scratch and cost about
20 us per camera frame over the frame's GEMMs).  The GEMM cores and the fused
Swin kernels also keep their LDS within the 160 KiB of a CU.
"""

import json
import pathlib

import pytest

REPORT = pathlib.Path(__file__).resolve().parent.parent / "bevfusion.c_amd" / "_build" / \
    "kernel_resources.json"


@pytest.fixture(scope="module")
def report():
    if not REPORT.exists():
        pytest.fail(f"{REPORT} missing: run __graft_entry__.build()")
    return json.loads(REPORT.read_text())


def test_every_source_reports_its_kernels(report):
    assert {"swin.hip", "camera.hip", "ops.hip", "bev.hip", "lss.hip"} <= set(report)
    assert sum(len(v) for v in report.values()) > 200
    gemm = [k for v in report.values() for k in v if "gemm_" in k]
    assert len(gemm) > 60


def test_no_scratch_or_vgpr_spills(report):
    bad = [(src, name, r) for src, kernels in report.items() for name, r in kernels.items()
           if r.get("scratch", 0) or r.get("vgpr_spill", 0)]
    assert not bad, bad[:5]


def test_hot_kernels_fit_lds(report):
    for src, kernels in report.items():
        for name, r in kernels.items():
            if any(s in name for s in ("gemm_", "swin_mlp", "window_msa", "window_attention")):
                assert r["lds"] <= 160 * 1024, (src, name, r["lds"])
                assert r["occupancy"] >= 1, (src, name)
