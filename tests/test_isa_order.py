"""Issue order of the streaming m = 1 kernels (gemv1.hip), checked on the compiled gfx950 assembly of this build.

The kernels stage activations and scales by LDS DMA, issue the first D weight-record loads, and then wait with a
hand-written `s_waitcnt vmcnt(D)`: loads retire in order, so that count covers exactly the DMAs. The count is only
right when the D record loads are issued before the wait; the compiler may move them (the records are read through a
restrict pointer, which an asm memory clobber does not order), and once it sank them into a branch behind the wait,
the B operands were read from LDS before the DMAs had landed. This test compiles gemv1.hip to assembly and checks, for
every instance of the whole-tile streaming kernels, that at least as many record loads as the wait's count precede
the first hand-written wait after the DMAs.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "qengine_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def first_wait(lines):
    """(count of the first s_waitcnt vmcnt after a DMA, DMAs before it, record loads before it), or None"""
    nlds = nrec = 0
    for l in lines:
        t = l.strip()
        if t.startswith("global_load_lds"):
            nlds += 1
        elif t.startswith("global_load_dword"):
            nrec += 1
        m = re.match(r"s_waitcnt vmcnt\((\d+)\)", t)
        if m and nlds > 0:
            return int(m.group(1)), nlds, nrec
    return None


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_record_loads_precede_the_dma_wait(tmp_path):
    asm = tmp_path / "gemv1.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-I", os.path.join(ROOT, "include"), "-I", CSRC, "--cuda-device-only", "-S", "-o",
           str(asm), os.path.join(CSRC, "gemv1.hip")]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    lines = asm.read_text().split("\n")
    starts = [n for n, l in enumerate(lines) if re.match(r"^_ZN8qe_gemv1\d+(gemv1s_kernel|gemv1s_w8c_kernel)\w*:", l)]
    assert len(starts) >= 20, len(starts)
    bad = []
    for st in starts:
        end = next(n for n in range(st, len(lines)) if lines[n].startswith(".Lfunc_end"))
        r = first_wait(lines[st:end])
        if r is None or r[2] < r[0]:
            bad.append((lines[st].split(":")[0], r))
    assert not bad, bad
