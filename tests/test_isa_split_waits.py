"""The small-M kernels split K over workgroups: each workgroup stores its
partial tile with agent-scope stores (global_store ... sc1), meets the other
waves at a barrier, and then one thread counts the workgroup in with an
atomic add; the last workgroup of a tile reads every partial back.  A
barrier orders instruction issue only, so every thread has to wait for its
own partial stores to be acknowledged (s_waitcnt vmcnt(0)) before that
barrier, or the counter can move while a partial is still in flight and the
last workgroup adds stale data.  This test disassembles the gfx950 code of
rq_smallm.hip and rq_smallm_codes.hip and checks, for every kernel with a split counter, that the
barrier before each counter atomic is reached with no agent-scope store
still unwaited."""
import re

import pytest

from tests.isa_util import HAVE_TOOLS, disassembly, kernels


def unwaited_counts(body):
    """Indices of counter atomics whose preceding barrier was reached while an
    agent-scope (sc1) global store issued since the last s_waitcnt vmcnt(0)
    may still have been in flight."""
    pending, barrier_pending, bad = False, False, []
    for i, ins in enumerate(body):
        op = ins.split()[0]
        if op.startswith("global_store") and re.search(r"\bsc1\b", ins):
            pending = True
        elif op == "s_waitcnt" and "vmcnt(0)" in ins:
            pending = False
        elif op == "s_barrier":
            barrier_pending = pending
        elif op.startswith("global_atomic_add") and barrier_pending:
            bad.append(i)
    return bad


def test_scan_flags_a_missing_wait():
    store = "global_store_dwordx2 v6, v[2:3], s[14:15] sc1"
    count = "global_atomic_add v2, v2, v3, s[18:19] sc0"
    assert unwaited_counts([store, "s_barrier", count]) == [2]
    assert unwaited_counts([store, "s_waitcnt vmcnt(0)", "s_barrier", count]) == []
    # a store after the count (the counter's reset) before a later barrier is
    # not the partials' store
    assert unwaited_counts([store, "s_waitcnt vmcnt(0)", "s_barrier", count, store, "s_barrier"]) == []


@pytest.mark.skipif(not HAVE_TOOLS, reason="ROCm toolchain not present")
def test_split_partials_complete_before_count(tmp_path):
    ks = kernels(disassembly("rq_smallm.hip", tmp_path), r"k_smallm")
    assert ks, "no k_smallm kernels in the code object"
    checked = set()
    for name, body in ks.items():
        if not any(ins.startswith("global_atomic_add") for ins in body):
            continue
        assert any(re.search(r"^global_store\S*\s.*\bsc1\b", ins) for ins in body), name
        base = "k_smallm_f32" if "k_smallm_f32" in name else "k_smallm_set" if "k_smallm_set" in name else "k_smallm"
        checked.add(base)
        bad = unwaited_counts(body)
        assert not bad, (name, [body[b] for b in bad[:3]])
    assert checked == {"k_smallm", "k_smallm_set", "k_smallm_f32"}, checked


@pytest.mark.skipif(not HAVE_TOOLS, reason="ROCm toolchain not present")
def test_codes_split_partials_complete_before_count(tmp_path):
    ks = kernels(disassembly("rq_smallm_codes.hip", tmp_path), r"k_smallm_codes")
    assert ks, "no k_smallm_codes kernels in the code object"
    checked = set()
    for name, body in ks.items():
        if not any(ins.startswith("global_atomic_add") for ins in body):
            continue
        assert any(re.search(r"^global_store\S*\s.*\bsc1\b", ins) for ins in body), name
        checked.add("k_smallm_codes_set" if "k_smallm_codes_set" in name else "k_smallm_codes")
        bad = unwaited_counts(body)
        assert not bad, (name, [body[b] for b in bad[:3]])
    assert checked == {"k_smallm_codes", "k_smallm_codes_set"}, checked
