"""Concurrent calls from several host threads, each on its own stream and its
own weight handle, as the reference's serving loop issues them (requests run
on a blocking pool, up to four at once: runtime1.rs:23, runtime1.rs:217).
Every result must equal the same call made alone, bit for bit: the kernels
are deterministic, the split-K partials and tile counters live in the calling
stream's own workspace (one buffer and counter block per device and stream,
held by one call at a time while it enqueues), and the library keeps no
mutable state shared between calls on different streams."""
import threading

import pytest
import torch

from runtimed_amd import rq, synth

pytestmark = pytest.mark.gpu


def _weight(qtype, n, k, seed):
    return rq.QWeight(qtype, synth.weight_blocks(qtype, seed, n, k), n, k)


def test_concurrent_streams_match_serial(dev):
    g = torch.Generator().manual_seed(5)
    cases = [
        # M = 1 GEMV (f32)
        (_weight(rq.Q4_K, 4864, 896, 1), torch.randn((1, 896), generator=g)),
        # small-M matrix-core path (bf16)
        (_weight(rq.Q6_K, 2048, 2048, 2), torch.randn((8, 2048), generator=g).to(torch.bfloat16)),
        # tiled GEMM with K split over workgroups (stream-ordered partials)
        (_weight(rq.Q6_K, 2048, 8192, 3), torch.randn((300, 8192), generator=g).to(torch.bfloat16)),
        # pipelined 256 x 256 GEMM
        (_weight(rq.Q4_K, 32768, 256, 4), torch.randn((512, 256), generator=g).to(torch.bfloat16)),
        # two activation rows on the segment GEMV and on the team GEMV (bf16)
        (_weight(rq.Q4_K, 4864, 896, 5), torch.randn((2, 896), generator=g).to(torch.bfloat16)),
        (_weight(rq.Q4_K, 896, 4864, 6), torch.randn((2, 4864), generator=g).to(torch.bfloat16)),
        # three f32 rows on the segment GEMV's four row slots
        (_weight(rq.Q8_0, 896, 896, 7), torch.randn((3, 896), generator=g)),
    ]
    cases = [(w, x.to(dev)) for w, x in cases]
    serial = [w.forward(x) for w, x in cases]
    torch.cuda.synchronize()

    results, errors = [None] * len(cases), []

    def work(i):
        try:
            s = torch.cuda.Stream(dev)
            w, x = cases[i]
            with torch.cuda.stream(s):
                outs = [w.forward(x) for _ in range(8)]
            s.synchronize()
            results[i] = outs
        except Exception as e:  # surfaced below
            errors.append(e)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(cases))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i, outs in enumerate(results):
        for o in outs:
            assert torch.equal(o, serial[i]), i
