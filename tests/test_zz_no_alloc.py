"""rq_fp8_gemm_noalloc: the FP8 GEMM with its activation scratch in a fixed
array of the library instead of the stream's workspace.  Called through the
C ABI and compared with rq_fp8_gemm (same kernels, so bit for bit) on two
calls in a row, the second smaller, plus the size limit and the no-scratch
e4m3 path.  Device memory in use must not change across its calls."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from runtimed_amd import rq, synth
from tests.conftest import norm_err

pytestmark = pytest.mark.gpu

LIMIT = 16 << 20  # RQ_NOALLOC_SCRATCH_BYTES


def _problem(m, n, k, seed, dev):
    x = torch.from_numpy(synth.activations(seed, m, k)).to(torch.bfloat16).to(dev)
    wq = torch.from_numpy(oracle.fp8_encode_array(synth.fp8_weight_values(seed + 1, n, k))).to(dev)
    ws = torch.from_numpy(synth.fp8_row_scales(seed + 2, n)).to(dev)
    return x, wq, ws


def _noalloc(x, xtype, m, wq, ws, n, k, y, mode=rq.FP8_PER_TOKEN):
    return rq.lib().rq_fp8_gemm_noalloc(rq._ptr(x), xtype, m, rq._ptr(wq), rq._ptr(ws), n, k, rq._ptr(y),
                                        rq.ftype(y.dtype), mode, rq._stream(y.device))


def _check(x, wq, ws, ydt=torch.bfloat16):
    m, k = x.shape
    n = wq.shape[0]
    y = torch.full((m, n), float("nan"), dtype=ydt, device=x.device)
    rq.check(_noalloc(x, rq.BF16, m, wq, ws, n, k, y))
    ref = rq.fp8_gemm(x, wq, ws, mode=rq.FP8_PER_TOKEN, out_dtype=ydt)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    return y


def test_noalloc_matches_fp8_gemm_twice_then_smaller(dev):
    # the FP8 workload (2048 x 14336 x 4096: 8 MiB + 8 KiB of scratch), then
    # a smaller call that reuses the array with stale bytes past its end
    print("noalloc fp8 2048x14336x4096 then 300x1000x640", flush=True)
    x, wq, ws = _problem(2048, 14336, 4096, 11, dev)
    y = _check(x, wq, ws)
    rows = np.array([0, 1, 1023, 2047])
    xq, xs = oracle.fp8_quantize_rows(x[rows].float().cpu().numpy())
    r = oracle.fp8_gemm_quantized_f64(xq, xs, wq.cpu().numpy(), ws.cpu().numpy())
    assert norm_err(y[rows].float().cpu().numpy(), r) <= 2e-2
    x2, wq2, ws2 = _problem(300, 1000, 640, 21, dev)
    _check(x2, wq2, ws2, torch.float32)
    _check(x, wq, ws)


def test_noalloc_allocates_nothing(dev):
    x, wq, ws = _problem(512, 4096, 2048, 31, dev)
    y = torch.empty((512, 4096), dtype=torch.bfloat16, device=dev)
    rq.check(_noalloc(x, rq.BF16, 512, wq, ws, 4096, 2048, y))  # the code object is loaded by now
    s = torch.cuda.Stream()  # a stream the workspace has never seen
    with torch.cuda.stream(s):
        y.zero_()  # HIP sets up the stream's queue at its first launch
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    with torch.cuda.stream(s):
        for _ in range(3):
            rq.check(_noalloc(x, rq.BF16, 512, wq, ws, 4096, 2048, y))
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0


def test_noalloc_limit_and_codes(dev):
    k, n = 4096, 256
    m_max = (LIMIT // (k + 4)) // 256 * 256
    x, wq, ws = _problem(m_max + 256, n, k, 41, dev)
    y = torch.full((m_max + 256, n), 7.0, device=dev)
    rc = _noalloc(x, rq.BF16, m_max + 256, wq, ws, n, k, y)
    assert rc == -5 and "scratch" in rq.lib().rq_last_error().decode()
    torch.cuda.synchronize()
    assert bool(torch.all(y == 7.0))  # nothing launched
    _check(x[:m_max].contiguous(), wq, ws, torch.float32)
    # e4m3 activations are used as they are: no scratch, any size
    xq = torch.from_numpy(oracle.fp8_encode_array(synth.fp8_weight_values(42, m_max + 256, k))).to(dev)
    yq = torch.empty((m_max + 256, n), dtype=torch.float32, device=dev)
    rq.check(_noalloc(xq, rq.F8E4M3, m_max + 256, wq, ws, n, k, yq))
    ref = rq.fp8_gemm(xq, wq, ws, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(yq, ref)
    # argument checks answer before any device work
    assert _noalloc(x, 99, 4, wq, ws, n, k, y) == -5
    assert rq.lib().rq_fp8_gemm_noalloc(None, rq.BF16, 0, None, None, n, k, None, rq.F32, 1, None) == 0
