"""Build recipe for the native libraries (invoked by __graft_entry__.build()).

Products (in-tree, next to their sources, so they travel with the tree):
  bevfusion.c_amd/lib/libbfmodel.so  BFW checkpoint and BFI frame readers (C11, gcc)
  bevfusion.c_amd/lib/libbfhip.so    gfx950 HIP kernels + the C-ABI entry points
Test infrastructure (built by the same call, never linked by the products):
  oracle/_build/liboracle*.so        CPU restatement of the reference path
  oracle/_ref/libbfref*.so           reference CPU sources, when /root/reference exists
"""

from __future__ import annotations

import concurrent.futures as cf
import json
import os
import pathlib
import re
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
OBJ = PKG / "_build"
INCLUDE = ROOT / "include"
ARCH = os.environ.get("BFHIP_ARCH", "gfx950")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # Packed-fp32 VALU forms are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: epilogues and softmax read them without
    # v_accvgpr_read copies.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def _run(cmd, quiet_packed=True):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines()
                    if not (quiet_packed and "packed-fp32-ops" in line))
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(map(str, cmd))}\n{out}")
    return out


def build_model_lib() -> pathlib.Path:
    LIB.mkdir(exist_ok=True)
    out = LIB / "libbfmodel.so"
    _run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-Wextra", f"-I{INCLUDE}",
          str(CSRC / "bfw_model.c"), str(CSRC / "bfi_frame.c"), "-o", str(out)])
    return out


_REMARK = re.compile(r"remark: +(Function Name|TotalSGPRs|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|"
                     r"Occupancy \[waves/SIMD\]|SGPRs Spill|VGPRs Spill|LDS Size \[bytes/block\]): "
                     r"(\S+) \[-Rpass-analysis=kernel-resource-usage\]")
_RESOURCE_KEYS = {"TotalSGPRs": "sgprs", "VGPRs": "vgprs", "AGPRs": "agprs",
                  "ScratchSize [bytes/lane]": "scratch", "Occupancy [waves/SIMD]": "occupancy",
                  "SGPRs Spill": "sgpr_spill", "VGPRs Spill": "vgpr_spill",
                  "LDS Size [bytes/block]": "lds"}


def _kernel_resources(text: str) -> dict:
    """Per-kernel resource usage from the compiler's kernel-resource-usage
    remarks: {mangled name: {sgprs, vgprs, agprs, scratch, occupancy,
    sgpr_spill, vgpr_spill, lds}}."""
    out, cur = {}, None
    for key, value in _REMARK.findall(text):
        if key == "Function Name":
            cur = out.setdefault(value, {})
        elif cur is not None:
            cur[_RESOURCE_KEYS[key]] = int(value)
    return out


def _compile_hip(src: pathlib.Path):
    OBJ.mkdir(exist_ok=True)
    obj = OBJ / (src.stem + ".o")
    text = _run([HIPCC, *HIP_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", str(src),
                 "-o", str(obj)])
    return obj, _kernel_resources(text)


def build_hip_lib(jobs: int | None = None) -> pathlib.Path:
    model = build_model_lib()
    sources = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 2) // 2))
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        built = list(pool.map(_compile_hip, sources))
    objs = [o for o, _ in built]
    # Kernel resource report (registers, scratch, occupancy, LDS) of every
    # kernel in the library, read by tests/test_kernel_resources.py.
    report = {src.name: res for src, (_, res) in zip(sources, built)}
    (OBJ / "kernel_resources.json").write_text(json.dumps(report, indent=1, sort_keys=True))
    out = LIB / "libbfhip.so"
    tmp = LIB / "libbfhip.so.tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs),
          f"-L{LIB}", "-lbfmodel", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)])
    tmp.replace(out)
    return out


def build_oracle(reference: str = "/root/reference") -> None:
    oracle = ROOT / "oracle"
    _run(["make", "-s", "-B", "-C", str(oracle), "oracle"])
    if pathlib.Path(reference, "src", "kernels_ref.c").exists():
        _run(["make", "-s", "-B", "-C", str(oracle), "ref", f"REF={reference}"])


def build_all() -> None:
    build_hip_lib()
    build_oracle()


if __name__ == "__main__":
    build_all()
    print("built", LIB / "libbfhip.so", file=sys.stderr)
