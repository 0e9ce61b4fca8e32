"""Paged-KV block quantizer on the device (cache/paged/quantize.rs): codes
and per-head scales bit-exact against the oracle for FP8 and INT8, the
decode bit-exact in f32 (and equal to the rounded f32 result in f16 /
bf16), the F16 sink path equal to a round-to-nearest-even cast, and the
reference's own tests (quantize.rs:142-200)."""
import numpy as np
import pytest
import torch

import oracle
from runtimed_amd import rq

pytestmark = pytest.mark.gpu

SHAPES = [(1, 8, 16, 128), (2, 4, 33, 64), (1, 2, 2, 16), (3, 1, 5, 7), (1, 8, 4096, 128), (2, 2, 700, 96)]
TDTYPES = [torch.float32, torch.float16, torch.bfloat16]


def rand_kv(shape, dtype, seed, specials=False):
    rng = np.random.default_rng(seed)
    t = (rng.standard_normal(shape) * rng.uniform(0.1, 4.0)).astype(np.float32)
    if specials:
        flat = t.reshape(-1)
        idx = rng.choice(flat.size, size=min(8, flat.size), replace=False)
        flat[idx[:2]] = np.nan
        flat[idx[2:4]] = 0.0
        flat[idx[4:6]] = -0.0
    return torch.from_numpy(t).to(dtype)


@pytest.mark.parametrize("int8", [False, True])
@pytest.mark.parametrize("dtype", TDTYPES)
@pytest.mark.parametrize("shape", SHAPES)
def test_quantize_bit_exact(dev, int8, dtype, shape):
    t = rand_kv(shape, dtype, sum(shape) + int8, specials=True)
    q, s = (rq.quantize_int8 if int8 else rq.quantize_fp8)(t.to(dev))
    want_q, want_s = oracle.kv_quantize(t.float().numpy(), int8)
    assert tuple(s.shape) == (1, shape[1], 1, 1)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), want_s.view(np.uint32))
    assert np.array_equal(q.cpu().view(torch.uint8).numpy(), want_q)


@pytest.mark.parametrize("int8", [False, True])
@pytest.mark.parametrize("shape", [(1, 8, 16, 128), (2, 3, 9, 40), (64,)])
def test_dequantize(dev, int8, shape):
    rng = np.random.default_rng(len(shape) + int8)
    codes = rng.integers(0, 256, shape, dtype=np.uint8)
    h = shape[1] if len(shape) == 4 else 1
    s = rng.uniform(1e-4, 0.05, h).astype(np.float32)
    qt = torch.from_numpy(codes).to(dev)
    if not int8:
        qt = qt.view(torch.float8_e4m3fn)
    deq = rq.dequantize_int8 if int8 else rq.dequantize_fp8
    want = oracle.kv_dequantize(codes, s, int8)
    got = deq(qt, torch.from_numpy(s).reshape(1, h, 1, 1).to(dev), torch.float32).cpu().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    for dt in (torch.float16, torch.bfloat16):
        got = deq(qt, torch.from_numpy(s).reshape(1, h, 1, 1).to(dev), dt).cpu()
        ref = torch.from_numpy(want).to(dt)
        assert torch.equal(torch.isnan(got), torch.isnan(ref))
        assert torch.equal(got[~torch.isnan(got)], ref[~torch.isnan(ref)])


@pytest.mark.parametrize("dtype", TDTYPES)
def test_f16_sink_cast(dev, dtype):
    t = rand_kv((1, 4, 16, 64), dtype, 5)
    kq, vq, ks, vs, prec = rq.quantize_block_kv(3, t.to(dev), t.to(dev), rq.KV_FP8)
    assert prec == rq.KV_F16 and kq.dtype == torch.float16 and vq.dtype == torch.float16
    assert torch.equal(kq.cpu(), t.to(torch.float16))
    assert ks.cpu().tolist() == [1.0] and vs.cpu().tolist() == [1.0]
    back = rq.dequantize_block(kq, ks, prec, torch.float32)
    assert torch.equal(back.cpu(), t.to(torch.float16).float())


def test_reference_tests(dev):  # quantize.rs:142-200
    data = torch.tensor([(i - 32.0) * 0.1 for i in range(64)]).reshape(1, 2, 2, 16).to(dev)
    q, s = rq.quantize_fp8(data)
    assert q.dtype == torch.float8_e4m3fn and tuple(s.shape) == (1, 2, 1, 1)
    assert torch.all((rq.dequantize_fp8(q, s, torch.float32) - data).abs() < 0.2)
    q, s = rq.quantize_int8(data)
    assert q.dtype == torch.uint8 and tuple(s.shape) == (1, 2, 1, 1)
    assert torch.all((rq.dequantize_int8(q, s, torch.float32) - data).abs() < 0.2)
    data = torch.tensor([i * 0.05 for i in range(64)]).reshape(1, 2, 2, 16).to(dev)
    q, s = rq.quantize_fp8(data)
    assert torch.all((rq.dequantize_fp8(q, s, torch.float32) - data).abs() < 0.2)
    zeros = torch.zeros((1, 2, 4, 16), device=dev)
    _, _, _, _, prec = rq.quantize_block_kv(0, zeros, zeros, rq.KV_FP8)
    assert prec == rq.KV_F16
    kq, vq, _, _, prec = rq.quantize_block_kv(16, zeros, zeros, rq.KV_FP8)
    assert prec == rq.KV_FP8 and kq.dtype == torch.float8_e4m3fn and vq.dtype == torch.float8_e4m3fn
    kq, _, ks, _, prec = rq.quantize_block_kv(16, zeros, zeros, rq.KV_INT8)
    assert prec == rq.KV_INT8 and kq.dtype == torch.uint8
    assert ks.reshape(-1).cpu().tolist() == [np.float32(1e-8)] * 2


def test_empty_and_errors(dev):
    s = torch.empty(3, device=dev)
    rq.check(rq.lib().rq_kv_quantize(None, rq.F32, 0, 3, 16, rq.KV_FP8, None, rq._ptr(s), None))
    torch.cuda.synchronize()
    assert s.cpu().tolist() == [np.float32(1e-8)] * 3
    with pytest.raises(rq.RqError) as e:
        rq.check(rq.lib().rq_kv_quantize(None, rq.F32, 1, 1, 1, 7, None, rq._ptr(s), None))
    assert e.value.code == -5


def test_empty_shape_under_graph_capture(dev):
    # the floor scales of an empty chunk come from a kernel, so the call can
    # be captured; every replay rewrites them (the eager fill between
    # replays puts other values there first)
    s8 = torch.empty(5, device=dev)
    s16 = torch.empty(5, device=dev)
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            h = torch.cuda.current_stream().cuda_stream
            rq.check(rq.lib().rq_kv_quantize(None, rq.F32, 1, 5, 0, rq.KV_INT8, None, rq._ptr(s8), h))
            rq.check(rq.lib().rq_kv_quantize(None, rq.BF16, 0, 5, 64, rq.KV_F16, None, rq._ptr(s16), h))
    for rep in range(3):
        s8.fill_(3.0 + rep)
        s16.fill_(-1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert s8.cpu().tolist() == [np.float32(1e-8)] * 5, rep
        assert s16.cpu().tolist() == [1.0] * 5, rep
    with pytest.raises(rq.RqError) as e:
        rq.check(rq.lib().rq_kv_dequantize(None, rq.KV_FP8, None, 1, 1, 4, None, rq.F32, None))
    assert e.value.code == -5
