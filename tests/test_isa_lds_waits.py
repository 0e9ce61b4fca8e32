"""The pipelined FP8 and quantized bf16 GEMMs issue their LDS fragment reads
as explicit ds_read_b128 instructions and complete them with one explicit
s_waitcnt lgkmcnt(0) (the compiler cannot see these reads, so it cannot
order their uses); the compiler's own LDS reads (the staged epilogues)
complete at its lgkmcnt(N) waits.  This test disassembles the gfx950 code of rq_fp8.hip
and rq_gemm.hip and checks, instruction by instruction, that no register written by
such a read is read or overwritten before the wait that completes it: a
register copied or reused early would hold stale data, or be clobbered when
the read lands."""
import re

import pytest

from tests.isa_util import HAVE_TOOLS, disassembly, kernels


def _regs(text: str) -> set:
    out = set()
    for m in re.finditer(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b", text):
        if m.group(1):
            out |= {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
        else:
            out.add(f"{m.group(4)}{m.group(5)}")
    return out


def early_uses(body):
    """(index, instruction) pairs that touch a register of an LDS read still
    in flight.  LDS operations (reads and writes) retire in issue order:
    `s_waitcnt lgkmcnt(N)` completes all but the newest N of them.  A scalar
    memory load shares that counter and may return out of order, so while
    one is outstanding only lgkmcnt(0) is taken to complete anything."""
    pending, bad, reads, smem = [], [], 0, False  # pending: register sets of LDS ops in issue order
    for ln, ins in enumerate(body):
        op = ins.split()[0]
        if op == "s_endpgm":
            break
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", ins)
            if m:
                keep = int(m.group(1))
                if keep == 0:
                    pending, smem = [], False
                elif not smem:
                    pending = pending[len(pending) - keep:] if len(pending) > keep else pending
            continue
        if op.startswith("s_load") or op.startswith("s_buffer_load"):
            smem = True
            continue
        if op.startswith("s_"):
            continue
        operands = ins[len(op):]
        live = set().union(*pending) if pending else set()
        if _regs(operands) & live:
            bad.append((ln, ins))
        if op.startswith("ds_read"):
            reads += 1
            pending.append(_regs(operands.split(",")[0]))
        elif op.startswith("ds_"):
            pending.append(set())
    return bad, reads


def test_scan_flags_an_early_use():
    body = ["ds_read_b128 v[4:7], v1", "v_mov_b32 v9, v5", "s_waitcnt lgkmcnt(0)", "v_mov_b32 v9, v5", "s_endpgm"]
    bad, reads = early_uses(body)
    assert reads == 1 and [b[0] for b in bad] == [1]


def test_scan_partial_waits_retire_oldest_first():
    body = ["ds_read_b128 v[4:7], v1", "ds_read_b128 v[8:11], v2", "s_waitcnt lgkmcnt(1)",
            "v_mov_b32 v20, v5",   # first read done
            "v_mov_b32 v21, v9",   # second still in flight
            "s_load_dword s4, s[0:1], 0x0", "ds_read_b32 v12, v3", "s_waitcnt lgkmcnt(1)",
            "v_mov_b32 v22, v12",  # a scalar load is outstanding: nothing retired
            "s_waitcnt lgkmcnt(0)", "v_mov_b32 v23, v12", "s_endpgm"]
    bad, reads = early_uses(body)
    assert reads == 3 and [b[0] for b in bad] == [4, 8]


def _check(tmp_path, src: str, pattern: str, min_reads: int):
    ks = kernels(disassembly(src, tmp_path), pattern)
    assert ks, f"{pattern} not found in the code object"
    for kern, body in ks.items():
        bad, reads = early_uses(body)
        assert reads >= min_reads, (kern, reads)
        assert not bad, (kern, bad[:5])


@pytest.mark.skipif(not HAVE_TOOLS, reason="ROCm toolchain not present")
def test_fp8_pipe_lds_reads_complete_before_use(tmp_path):
    _check(tmp_path, "rq_fp8.hip", "k_fp8_gemm_pipe", 16)


@pytest.mark.skipif(not HAVE_TOOLS, reason="ROCm toolchain not present")
def test_qgemm_pipe_lds_reads_complete_before_use(tmp_path):
    # one eight-wave kernel per GGUF format; 6 reads of the first pass plus 12 per step
    _check(tmp_path, "rq_gemm.hip", "k_qgemm_pipe8", 18)


@pytest.mark.skipif(not HAVE_TOOLS, reason="ROCm toolchain not present")
def test_q6_pipe_lds_reads_complete_before_use(tmp_path):
    # the eight-wave Q6_K chunk-pair kernel: reads at base registers plus
    # offsets, 6 of the first pass plus 12 per step
    _check(tmp_path, "rq_gemm.hip", "k_q6_pipe8", 18)
