"""The layer GEMMs issue their MFMAs (dense v_mfma and 2:4-sparse v_smfmac) from inline asm (to hold a fixed issue
order), which the compiler's hazard recognizer does not see. The VALU promotion of a block partial, and code the
compiler places after the K loop, must not read an MFMA's result before the matrix core has written it; and no VALU
instruction may write a register an MFMA reads (the sparse MFMA's zeroed accumulator above all) too shortly before it.
This test compiles the kernels that use the asm MFMAs to gfx950 assembly and checks both against the wait states hipcc
itself inserts around the same instructions in one-MFMA probe kernels. CPU only."""
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


def _early_reads(lines, need, prefix="v_mfma"):
    """(line, instruction) of VALU reads of the destination VGPRs of an MFMA (instructions starting with `prefix`)
    fewer than `need` wait states after it."""
    out = []
    for i, line in enumerate(lines):
        s = line.strip()
        if not s.startswith(prefix):
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
            if t.startswith(("v_mfma", "v_smfmac")) or not t.startswith("v_"):
                continue
            ops = re.findall(r"v\[\d+:\d+\]|v\d+\b", t.split(None, 1)[1] if " " in t else "")
            srcs = set().union(*[_regs(o) for o in ops[1:]]) if len(ops) > 1 else set()
            if dst & srcs:
                out.append((j, t))
    return out


def _late_writes(lines, need):
    """(line, instruction) of VALU writes of a VGPR that a v_mfma or v_smfmac reads (its sources, and the sparse
    MFMA's accumulator, which is also its destination) fewer than `need` wait states before it."""
    out = []
    for i, line in enumerate(lines):
        s = line.strip()
        if not s.startswith(("v_mfma", "v_smfmac")):
            continue
        ops = [o.strip() for o in s.split(None, 1)[1].split(",")]
        reads = set().union(*[_regs(o) for o in (ops if s.startswith("v_smfmac") else ops[1:])])
        ws, j = 0, i - 1
        while j >= 0 and ws < need:
            t = lines[j].strip()
            j -= 1
            if not t or t.startswith(";") or t.startswith("."):
                continue
            if t.startswith("s_nop"):
                ws += int(t.split()[1]) + 1
                continue
            if t.startswith("v_") and not t.startswith(("v_mfma", "v_smfmac")) and " " in t:
                if _regs(t.split(None, 1)[1].split(",")[0].strip()) & reads:
                    out.append((j + 2, t))
            ws += 1
    return out


FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Xclang", "-target-feature",
         "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S"]

PROBE = r"""
#include <hip/hip_runtime.h>
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
__global__ void probe(const v8i *a, const v8i *b, float *o, float s)
{
    v4f z = {0.f, 0.f, 0.f, 0.f};
    v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[threadIdx.x], b[threadIdx.x], z, 0, 0, 0, 0, 0, 0);
    o[threadIdx.x] = __builtin_fmaf(p[0], s, p[1]);
}
"""


def _compiler_wait_states(tmp_path):
    src = tmp_path / "probe.hip"
    src.write_text(PROBE)
    asm = tmp_path / "probe.s"
    r = subprocess.run([HIPCC] + FLAGS + [str(src), "-o", str(asm)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [x.strip() for x in asm.read_text().splitlines()]
    i = next(k for k, x in enumerate(lines) if x.startswith("v_mfma_f32_16x16x128_f8f6f4"))
    nop = lines[i + 1]
    assert nop.startswith("s_nop"), f"expected the compiler's s_nop after the probe MFMA, got {nop!r}"
    return int(nop.split()[1]) + 1


PROBE_SP = r"""
#include <hip/hip_runtime.h>
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
__global__ void probe_read(const v4i *a, const v8i *b, const int *x, float *o, float s)
{
    v4f z = {0.f, 0.f, 0.f, 0.f};
    v4f p = __builtin_amdgcn_smfmac_f32_16x16x128_fp8_fp8(a[threadIdx.x], b[threadIdx.x], z, x[threadIdx.x], 0, 0);
    o[threadIdx.x] = __builtin_fmaf(p[0], s, p[1]);
}
__global__ void probe_write(const v4i *a, const v8i *b, const int *x, const float *c, float *o)
{
    const float t = c[threadIdx.x];
    v4f z = {t * t, t * t, t * t, t * t};
    v4f p = __builtin_amdgcn_smfmac_f32_16x16x128_fp8_fp8(a[threadIdx.x], b[threadIdx.x], z, x[threadIdx.x], 0, 0);
    o[threadIdx.x] = p[0] + p[1] + p[2] + p[3];
}
"""


def _compiler_sparse_wait_states(tmp_path):
    """(wait states from a v_smfmac to a VALU read of its result, from a VALU write of its accumulator to it), as hipcc
    places them in the probe kernels."""
    src = tmp_path / "probe_sp.hip"
    src.write_text(PROBE_SP)
    asm = tmp_path / "probe_sp.s"
    r = subprocess.run([HIPCC] + FLAGS + [str(src), "-o", str(asm)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [x.split(";")[0].strip() for x in asm.read_text().splitlines()]
    lines = [x for x in lines if x and not x.startswith(".")]
    sm = [k for k, x in enumerate(lines) if x.startswith("v_smfmac")]
    assert len(sm) == 2, sm
    nop = lines[sm[0] + 1]
    assert nop.startswith("s_nop"), f"expected the compiler's s_nop after the probe's sparse MFMA, got {nop!r}"
    need_read = int(nop.split()[1]) + 1
    acc = _regs(lines[sm[1]].split(None, 1)[1].split(",")[0].strip())
    ws, j = 0, sm[1] - 1
    while not (lines[j].startswith("v_") and _regs(lines[j].split(None, 1)[1].split(",")[0].strip()) & acc):
        ws += int(lines[j].split()[1]) + 1 if lines[j].startswith("s_nop") else 1
        j -= 1
    return need_read, ws


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src", ["layer.hip", "quant.hip"])
def test_sparse_mfma_hazards(tmp_path, src):
    """The asm v_smfmac of the 2:4-sparse K step: no VALU read of its result, and no VALU write of a register it reads,
    closer to it than hipcc places them around the builtin."""
    need_read, need_write = _compiler_sparse_wait_states(tmp_path)
    assert need_read >= 4 and need_write >= 2, (need_read, need_write)
    asm = tmp_path / (src + ".s")
    cmd = [HIPCC] + FLAGS + ["-I" + os.path.join(os.path.dirname(CSRC), "..", "include"), "-I" + CSRC,
                             os.path.join(CSRC, src), "-o", str(asm)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = asm.read_text().splitlines()
    assert sum(1 for x in lines if x.strip().startswith("v_smfmac")) > 0
    bad = _early_reads(lines, need_read, "v_smfmac")
    assert not bad, f"VALU reads of sparse MFMA results too early in {src} (need {need_read}): {bad[:5]}"
    bad = _late_writes(lines, need_write)
    assert not bad, f"VALU writes too close before an MFMA that reads them in {src} (need {need_write}): {bad[:5]}"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src", ["layer.hip", "px.hip", "quant.hip"])
def test_no_early_accumulator_reads(tmp_path, src):
    need = _compiler_wait_states(tmp_path)
    assert need >= 11
    asm = tmp_path / (src + ".s")
    cmd = [HIPCC] + FLAGS + ["-I" + os.path.join(os.path.dirname(CSRC), "..", "include"), "-I" + CSRC,
                             os.path.join(CSRC, src), "-o", str(asm)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = asm.read_text().splitlines()
    assert sum(1 for x in lines if x.strip().startswith("v_mfma")) > 0
    bad = _early_reads(lines, need)
    assert not bad, f"VALU reads of MFMA results too early in {src} (need {need} wait states): {bad[:5]}"


def _resources(tmp_path, src):
    """{kernel: (VGPRs, VGPR spills, scratch bytes per lane)} from hipcc's resource-usage remarks."""
    r = subprocess.run([HIPCC] + FLAGS[:-1] + ["-c", "-I" + os.path.join(os.path.dirname(CSRC), "..", "include"),
                                                "-I" + CSRC, os.path.join(CSRC, src), "-o", str(tmp_path / "k.o"),
                                                "-Rpass-analysis=kernel-resource-usage"],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    out, cur = {}, None
    for line in r.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
            out[cur] = [None, None, None]
        for i, key in enumerate((r"VGPRs: (\d+)", r"VGPRs Spill: (\d+)", r"ScratchSize \[bytes/lane\]: (\d+)")):
            m = re.search(key, line)
            if m and cur:
                out[cur][i] = int(m.group(1))
    return out


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src", ["layer.hip", "px.hip", "quant.hip", "attn.hip", "norm.hip"])
def test_no_scratch(tmp_path, src):
    """No kernel spills registers or keeps an array in scratch memory: a dynamically indexed accumulator array, or
    two main loops whose registers the allocator cannot keep apart, silently moves the accumulators to memory and
    slows the kernel several times over."""
    res = _resources(tmp_path, src)
    assert res
    bad = {k: v for k, v in res.items() if v[1] or v[2]}
    assert not bad, f"kernels with spills or scratch in {src}: {bad}"

