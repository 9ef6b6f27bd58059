"""The host file readers under AddressSanitizer + UndefinedBehaviorSanitizer.

The BFW checkpoint reader (bevfusion.c_amd/csrc/bfw_model.c) and the BFI
frame reader (bfi_frame.c) parse untrusted files.  This test compiles them
with gcc, -fsanitize=address,undefined and -fno-sanitize-recover, together
with the driver tests/san_readers.c, and runs the driver over a corpus of
malformed files built from valid ones: every truncation point of the header
and directory, every header and directory byte overwritten (with the
directory / payload CRC recomputed, so the field checks behind the CRC run
too, and without), extreme values in every header field, and payload bytes
flipped.  The reference builds the same readers with ASan/UBSan
(CMakeLists.txt:179-194) and runs its container tests under them
(runs/rtx4060ti-2026-07-18/validation.txt:10-13).

Pass means: no sanitizer report and no leak (LeakSanitizer is on) over the
whole corpus, whether the reader accepts a file or not; truncated files and
unterminated names rejected at open; flipped payload bytes caught by
validation; the unmodified files open and validate; and over a thousand of
the BFW cases rejected, so the corpus reaches the reader's rejection paths.
Only the host C readers are built this way: the create-time checks of the
HIP contexts are compiled by hipcc into the GPU library and are covered by
the invalid-contract cases of test_abi.py instead.
"""

import os
import shutil
import struct
import subprocess
import zlib

import numpy as np
import pytest

from bfhip import bfw, frame_scene

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "bevfusion.c_amd", "csrc")
SAN_ENV = {
    "ASAN_OPTIONS": "detect_leaks=1:exitcode=86:verify_asan_link_order=0",
    "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1:exitcode=87",
}

pytestmark = pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    out = tmp_path_factory.mktemp("san") / "san_readers"
    cmd = ["gcc", "-std=c11", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-Wall", "-Werror", f"-I{os.path.join(ROOT, 'include')}",
           os.path.join(ROOT, "tests", "san_readers.c"), os.path.join(CSRC, "bfw_model.c"),
           os.path.join(CSRC, "bfi_frame.c"), "-lm", "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0 and ("asan" in r.stderr or "ubsan" in r.stderr):
        pytest.skip(f"sanitizer runtime not available: {r.stderr[-300:]}")
    assert r.returncode == 0, r.stderr
    return out


def _run(driver, kind, paths):
    env = dict(os.environ, **SAN_ENV)
    r = subprocess.run([str(driver), kind, *map(str, paths)], capture_output=True, text=True,
                       env=env, timeout=600)
    lines = r.stdout.splitlines()
    if r.returncode != 0:
        last = [l for l in lines if l.startswith("begin ")][-1:]
        pytest.fail(f"sanitizer stop (exit {r.returncode}) at {last}: {r.stderr[-3000:]}")
    status = {}
    for line in lines:
        word, _, rest = line.partition(" ")
        if word in ("ok", "invalid", "rejected"):
            status[rest.split(":")[0].split(" ")[0]] = (word, line)
    assert len(status) == len(paths), f"{len(status)} results for {len(paths)} files"
    return status


# ---------------------------------------------------------------- BFW files

def _bfw_base(path):
    r = np.random.default_rng(4)
    tensors = [("layer.weight", r.standard_normal((3, 5, 2)).astype(np.float32)),
               ("layer.index", np.arange(-3, 6, dtype=np.int64)),
               ("z", np.ones(1, np.float32))]
    bfw.write_bfw(tensors, path)
    return bytearray(path.read_bytes())


def _bfw_fix_crc(raw):
    """Recompute the directory CRC after a change inside the directory."""
    h = list(bfw.HEADER.unpack_from(raw, 0))
    count, dir_off = h[3], h[4]
    end = dir_off + count * bfw.ENTRY.size
    if 0 <= dir_off <= end <= len(raw) and count < 1 << 20:
        h[7] = zlib.crc32(bytes(raw[dir_off:end])) & 0xFFFFFFFF
        bfw.HEADER.pack_into(raw, 0, *h)
    return raw


def test_bfw_reader_under_sanitizers(driver, tmp_path):
    base_path = tmp_path / "base.bfw"
    base = _bfw_base(base_path)
    hdr = bfw.HEADER.unpack_from(base, 0)
    directory_end = hdr[4] + hdr[3] * bfw.ENTRY.size
    files = {}

    def add(name, raw):
        p = tmp_path / f"{name}.bfw"
        p.write_bytes(bytes(raw))
        files[p.name] = p

    for n in sorted({0, 1, 7, 8, 12, 63, 64, 65, directory_end - 1, directory_end,
                     hdr[5] - 1, hdr[5], len(base) - 1} | set(range(0, directory_end, 37))):
        add(f"trunc{n}", base[:n])
    for pos in range(directory_end):
        for val in (0x00, 0xFF, base[pos] ^ 0x80):
            raw = bytearray(base)
            raw[pos] = val
            add(f"byte{pos}_{val}", raw)
            if pos >= bfw.HEADER.size:
                add(f"bytecrc{pos}_{val}", _bfw_fix_crc(raw))
    # Header fields at boundary values (directory CRC stays valid).
    fields = [(8, "<I"), (12, "<I"), (16, "<Q"), (24, "<Q"), (32, "<Q"), (40, "<Q"),
              (48, "<I"), (52, "<I")]
    for off, fmt in fields:
        top = (1 << (8 * struct.calcsize(fmt))) - 1
        for v in (0, 1, 2, 63, 64, 65, len(base) - 1, len(base), len(base) + 1,
                  (top >> 1), (top >> 1) + 1, top):
            raw = bytearray(base)
            struct.pack_into(fmt, raw, off, v & top)
            add(f"field{off}_{v}", raw)
    # Directory entry fields at boundary values (CRC recomputed).
    for e in range(hdr[3]):
        at = hdr[4] + e * bfw.ENTRY.size
        for rel, fmt in [(96, "<I"), (100, "<I"), (104, "<I"), (108, "<I"), (132, "<I"),
                         (136, "<Q"), (144, "<Q"), (152, "<I"), (156, "<I")]:
            top = (1 << (8 * struct.calcsize(fmt))) - 1
            for v in (0, 1, 8, 9, 63, 64, len(base), (top >> 1) + 1, top):
                raw = bytearray(base)
                struct.pack_into(fmt, raw, at + rel, v & top)
                add(f"entry{e}_{rel}_{v}", _bfw_fix_crc(raw))
        raw = bytearray(base)
        raw[at:at + 96] = b"x" * 96            # name without a terminator
        add(f"noterm{e}", _bfw_fix_crc(raw))
    for pos in (hdr[5], hdr[5] + 5, len(base) - 1):
        raw = bytearray(base)
        raw[pos] ^= 0x01
        add(f"payload{pos}", raw)

    paths = [base_path] + list(files.values())
    status = _run(driver, "bfw", paths)
    word, line = status[str(base_path)]
    assert word == "ok" and " each 1 " in line, line
    for name, p in files.items():
        if name.startswith("payload"):
            assert status[str(p)][0] == "invalid", status[str(p)][1]
        elif name.startswith(("trunc", "noterm")):
            assert status[str(p)][0] == "rejected", status[str(p)][1]
    # Many overwritten bytes leave a valid file (name characters, unused dims
    # past the rank, flags, bytes already holding the written value); the
    # corpus must still drive the reader through its rejection paths.
    assert sum(w == "rejected" for w, _ in status.values()) > 1000


# ---------------------------------------------------------------- BFI files

def test_bfi_reader_under_sanitizers(driver, tmp_path):
    f = frame_scene.frame(seed=3, points=123)
    f["points"] = np.nan_to_num(f["points"], nan=0.5)
    base_path = tmp_path / "base.bfi"
    frame_scene.write_bfi(f, base_path)
    base = base_path.read_bytes()
    size = len(base)
    cases = []
    for n in (0, 4, 64, 127, 128, 129, size - 4, size - 1):
        cases.append((f"trunc{n}", lambda n=n: base[:n]))
    for off in range(4, 128, 4):
        for v in (0, 1, 0x7FFFFFFF, 0xFFFFFFFF):
            def mk(off=off, v=v):
                raw = bytearray(base)
                struct.pack_into("<I", raw, off, v)
                return raw
            cases.append((f"word{off}_{v}", mk))
    for off in (16, 24, 40, 48, 56, 64, 72, 80, 88):       # 64-bit sizes, counts, offsets
        for v in (size, size + 1, 1 << 62, (1 << 64) - 1, 124, 130):
            def mk(off=off, v=v):
                raw = bytearray(base)
                struct.pack_into("<Q", raw, off, v)
                return raw
            cases.append((f"quad{off}_{v}", mk))
    for pos in (128, 1000, size - 1):
        def mk(pos=pos):
            raw = bytearray(base)
            raw[pos] ^= 0x01                                # payload CRC no longer matches
            return raw
        cases.append((f"payload{pos}", mk))

    results = _run(driver, "bfi", [base_path])
    assert results[str(base_path)][0] == "ok", results[str(base_path)][1]
    batch = 12                                              # 13 MB files: a few at a time
    for i in range(0, len(cases), batch):
        paths = []
        for name, make in cases[i:i + batch]:
            p = tmp_path / f"{name}.bfi"
            p.write_bytes(bytes(make()))
            paths.append(p)
        status = _run(driver, "bfi", paths)
        for p in paths:
            if p.name.startswith(("trunc", "payload")):
                assert status[str(p)][0] == "rejected", status[str(p)][1]
            p.unlink()
