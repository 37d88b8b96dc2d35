"""The layer GEMMs issue their MFMAs from inline asm (to hold a fixed issue order), which the compiler's hazard
recognizer does not see. Code the compiler places after them (the epilogue, or a register copy where paths join) must
not read an accumulator with VALU before the matrix core has written it. This test compiles the kernels that use the
asm MFMAs to gfx950 assembly and checks that no VALU instruction reads a VGPR written by a v_mfma within 19 wait
states (the distance a 16-pass XDL result needs; the 16x16x128 FP8 MFMA is 8 passes and needs 11). CPU only."""
import os
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "xtagger_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _regs(spec):
    m = re.match(r"v\[(\d+):(\d+)\]", spec)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", spec)
    return {int(m.group(1))} if m else set()


def _early_reads(lines, need=19):
    """(line, instruction) of VALU reads of an MFMA's destination VGPRs fewer than `need` wait states after it."""
    out = []
    for i, line in enumerate(lines):
        s = line.strip()
        if not s.startswith("v_mfma"):
            continue
        dst = _regs(s.split()[1].rstrip(","))
        ws, j = 0, i + 1
        while j < len(lines) and ws < need:
            t = lines[j].strip()
            j += 1
            if not t or t.startswith(";") or t.startswith("."):
                continue
            if t.startswith("s_nop"):
                ws += int(t.split()[1]) + 1
                continue
            ws += 1
            if t.startswith("v_mfma") or not t.startswith("v_"):
                continue
            ops = re.findall(r"v\[\d+:\d+\]|v\d+\b", t.split(None, 1)[1] if " " in t else "")
            srcs = set().union(*[_regs(o) for o in ops[1:]]) if len(ops) > 1 else set()
            if dst & srcs:
                out.append((j, t))
    return out


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src", ["layer.hip", "px.hip"])
def test_no_early_accumulator_reads(tmp_path, src):
    asm = tmp_path / (src + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Xclang",
           "-target-feature", "-Xclang", "-packed-fp32-ops", "-I" + os.path.join(os.path.dirname(CSRC), "..", "include"),
           "-I" + CSRC, "--cuda-device-only", "-S", os.path.join(CSRC, src), "-o", str(asm)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    bad = _early_reads(asm.read_text().splitlines())
    assert not bad, f"VALU reads of MFMA results too early in {src}: {bad[:5]}"
