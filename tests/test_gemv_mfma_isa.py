"""ISA guard of the matrix-core GEMV (floyd_amd/csrc/gemv_mfma.hip), no GPU.

The kernel loads its x slice with inline-asm loads the compiler does not
track, issues the weight DMA, and only then waits (s_waitcnt vmcnt(ND)) and
reads the loaded registers.  That is correct only if no instruction between
a load and the wait touches its destination registers (a register copy
inserted by the allocator there would read data that has not landed).  This
compiles the file for gfx950 and checks every instantiation's code.
"""
import os
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(ROOT, "floyd_amd", "csrc", "gemv_mfma.hip")


def _hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    return path if os.path.exists(path) else None


def _regs(op):
    """VGPR numbers named by an operand text (v7, v[4:7])."""
    out = set()
    for a, b in re.findall(r"\bv\[(\d+):(\d+)\]", op):
        out.update(range(int(a), int(b) + 1))
    for a in re.findall(r"\bv(\d+)\b", op):
        out.add(int(a))
    return out


@pytest.mark.skipif(_hipcc() is None, reason="hipcc not available")
def test_untracked_x_loads_are_not_touched_before_their_wait(tmp_path):
    asm = tmp_path / "gemv_mfma.s"
    cmd = [_hipcc(), "--offload-arch=gfx950", "-O3", "-std=c++17", "--cuda-device-only", "-S",
           "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "floyd_amd", "csrc"),
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", SRC, "-o", str(asm)]
    subprocess.run(cmd, check=True, capture_output=True)
    lines = asm.read_text().splitlines()
    kernels = 0
    i = 0
    while i < len(lines):
        m = re.match(r"^(_Z\S*gemv_mfma_kernel\S*):", lines[i])
        if not m:
            i += 1
            continue
        kernels += 1
        name = m.group(1)
        j = i + 1
        pending = set()
        in_asm = False
        loads = 0
        checked = False
        while j < len(lines) and not lines[j].startswith(".Lfunc_end"):
            text = lines[j].strip()
            if text.startswith(";;#ASMSTART"):
                in_asm = True
            elif text.startswith(";;#ASMEND"):
                in_asm = False
            elif in_asm and text.startswith("global_load_dwordx4"):
                dst = text.split()[1].rstrip(",")
                pending |= _regs(dst)
                loads += 1
            elif in_asm and text.startswith("s_waitcnt vmcnt"):
                checked = True
                break
            elif text and not text.startswith(";") and not text.startswith(".") and pending:
                ops = text.split(None, 1)[1] if " " in text else ""
                touched = _regs(ops.split(";")[0]) & pending
                assert not touched, f"{name}: '{text}' touches in-flight v{sorted(touched)}"
            j += 1
        assert loads > 0 and checked, f"{name}: untracked loads / wait not found"
        i = j
    assert kernels >= 12
