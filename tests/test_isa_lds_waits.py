"""The pipelined FP8 and quantized bf16 GEMMs issue their LDS fragment reads
as explicit ds_read_b128 instructions and complete them with one explicit
s_waitcnt lgkmcnt(0) (the compiler cannot see these reads, so it cannot
order their uses).  This test compiles rq_fp8.hip and rq_gemm.hip to gfx950
assembly and checks, instruction by instruction, that no register written by
such a read is read or overwritten before the wait that completes it: a
register copied or reused early would hold stale data, or be clobbered when
the read lands."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = "/opt/rocm/bin/hipcc"


def _regs(text: str) -> set:
    out = set()
    for m in re.finditer(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b", text):
        if m.group(1):
            out |= {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
        else:
            out.add(f"{m.group(4)}{m.group(5)}")
    return out


def early_uses(lines, kernel: str):
    """(line, instruction) pairs that touch a register of an LDS read still in
    flight; reads retire at the next s_waitcnt lgkmcnt(0)."""
    start = next(i for i, l in enumerate(lines) if l.startswith(kernel + ":"))
    pending, bad, reads = {}, [], 0
    for ln in range(start + 1, len(lines)):
        ins = lines[ln].split(";")[0].strip()
        if not ins or ins.endswith(":") or ins.startswith("."):
            continue
        if ins.startswith("s_endpgm"):
            break
        op = ins.split()[0]
        if op == "s_waitcnt" and "lgkmcnt(0)" in ins:
            pending.clear()
            continue
        if op.startswith("s_"):
            continue
        operands = ins[len(op):]
        if _regs(operands) & set(pending):
            bad.append((ln, ins))
        if op.startswith("ds_read"):
            reads += 1
            for r in _regs(operands.split(",")[0]):
                pending[r] = ln
    return bad, reads


def test_scan_flags_an_early_use():
    lines = ["k:", "\tds_read_b128 v[4:7], v1", "\tv_mov_b32 v9, v5", "\ts_waitcnt lgkmcnt(0)",
             "\tv_mov_b32 v9, v5", "\ts_endpgm"]
    bad, reads = early_uses(lines, "k")
    assert reads == 1 and [b[0] for b in bad] == [2]


def _check(tmp_path, src: str, pattern: str, min_reads: int):
    out = tmp_path / (Path(src).stem + ".s")
    cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", "-x", "hip",
           str(ROOT / "runtimed_amd" / "csrc" / src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    lines = out.read_text().splitlines()
    kernels = [m.group(1) for l in lines if (m := re.match(r"^(_Z\S*" + pattern + r"\S*):", l))]
    assert kernels, f"{pattern} not found in the assembly"
    for kern in kernels:
        bad, reads = early_uses(lines, kern)
        assert reads >= min_reads, (kern, reads)
        assert not bad, (kern, bad[:5])


HAVE_HIPCC = shutil.which(HIPCC) is not None or Path(HIPCC).exists()


@pytest.mark.skipif(not HAVE_HIPCC, reason="hipcc not present")
def test_fp8_pipe_lds_reads_complete_before_use(tmp_path):
    _check(tmp_path, "rq_fp8.hip", "k_fp8_gemm_pipe", 16)


@pytest.mark.skipif(not HAVE_HIPCC, reason="hipcc not present")
def test_qgemm_pipe_lds_reads_complete_before_use(tmp_path):
    # one kernel per GGUF format; 8 reads of the first pass plus 16 per step
    _check(tmp_path, "rq_gemm.hip", "k_qgemm_pipe", 24)


@pytest.mark.skipif(not HAVE_HIPCC, reason="hipcc not present")
def test_q6_pipe_lds_reads_complete_before_use(tmp_path):
    # the Q6_K chunk-pair kernel: reads at base registers plus offsets
    _check(tmp_path, "rq_gemm.hip", "k_q6_pipe", 24)
