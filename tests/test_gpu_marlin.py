"""Marlin INT4 weights on the device (marlin_gemv.rs): repack and dequant
bit-exact against the oracle, the GEMV within normalized error 1e-3 of the
oracle's f64 product (f32 accumulation), and the reference's own tests
(marlin_gemv.rs:209-249, linear_layer.rs:143-185) through the C ABI."""
import numpy as np
import pytest
import torch

import oracle
from runtimed_amd import rq
from tests.conftest import norm_err

pytestmark = pytest.mark.gpu

WTYPES = [torch.float32, torch.float16, torch.bfloat16]


def packed_np(mw: rq.MarlinWeight) -> np.ndarray:
    return mw.packed.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("wdtype", WTYPES)
@pytest.mark.parametrize("n,k", [(32, 50), (7, 33), (96, 896), (4864, 896), (300, 4100)])
def test_repack_bit_exact(dev, wdtype, n, k):
    rng = np.random.default_rng(n * 7 + k)
    w = torch.from_numpy(rng.standard_normal((n, k)).astype(np.float32) * 2.5).to(wdtype)
    s = (rng.uniform(0.05, 0.6, n) * rng.choice([-1, 1], n)).astype(np.float32)
    mw = rq.repack_marlin_tiles(w.to(dev), torch.from_numpy(s).to(dev))
    want = oracle.marlin_repack(w.float().numpy(), s)
    assert tuple(mw.packed.shape) == want.shape
    assert np.array_equal(packed_np(mw), want)


def test_repack_special_values(dev):
    # exact ties (half away from zero), clamps, NaN / inf, the 1e-12 floor and
    # a NaN scale, all on one row each
    row = np.array([0.25, -0.25, 0.75, 1.25, -1.25, 50, -50, np.nan, np.inf, -np.inf, 0.0, -0.0],
                   np.float32)
    w = np.stack([row, row, row, row, row * 3])
    s = np.array([0.5, 0.0, 1e-13, np.nan, -0.75], np.float32)
    mw = rq.repack_marlin_tiles(torch.from_numpy(w).to(dev), torch.from_numpy(s).to(dev))
    assert np.array_equal(packed_np(mw), oracle.marlin_repack(w, s))


@pytest.mark.parametrize("n,k", [(32, 50), (5, 4), (64, 896), (1000, 4096)])
def test_dequant_bit_exact(dev, n, k):
    rng = np.random.default_rng(k)
    words = rng.integers(0, 2**32, ((k + 31) // 32, n, 4), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(-1, 1, n).astype(np.float32)
    mw = rq.MarlinWeight(torch.from_numpy(words.view(np.int32)).to(dev), torch.from_numpy(s).to(dev), k, n)
    got = mw.dequantize().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), oracle.marlin_dequant(words, s, k).view(np.uint32))


XTYPES = [(torch.float32, 1e-3), (torch.float16, 1e-3), (torch.bfloat16, 1e-2)]


@pytest.mark.parametrize("xdtype,tol", XTYPES)
@pytest.mark.parametrize("m,n,k", [(1, 4864, 896), (1, 896, 4864), (2, 32, 50), (3, 300, 100),
                                   (1, 128, 896), (5, 14336, 4096), (9, 40000, 64), (4, 33, 1000),
                                   (1, 14336, 4096), (1, 40000, 64), (1, 100, 15360), (1, 70, 1000),
                                   # M = 1 with n >= 8192 and n k >= 2^24 on the matrix cores: 4, 8 and 16 chunks a
                                   # wave, partial 32-row tiles, and (k = 2080) chunk slots past the end
                                   (1, 16400, 1024), (1, 8210, 4096), (1, 8200, 8192), (1, 8200, 2080)])
def test_gemv_parity(dev, xdtype, tol, m, n, k):
    rng = np.random.default_rng(m * 1000 + n + k)
    words = rng.integers(0, 2**32, ((k + 31) // 32, n, 4), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(0.001, 0.02, n).astype(np.float32)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(xdtype)
    mw = rq.MarlinWeight(torch.from_numpy(words.view(np.int32)).to(dev), torch.from_numpy(s).to(dev), k, n)
    y = rq.marlin_gemv(x.to(dev), mw)
    assert y.dtype == xdtype and tuple(y.shape) == (m, n)
    want = oracle.marlin_gemv_f64(x.float().numpy(), words, s)
    # f32 accumulation: 1e-3; a bf16 output adds its own rounding (2^-8)
    assert norm_err(y.float().cpu().numpy(), want) < tol


def test_reference_cuda_test(dev):  # marlin_gemv.rs:224-249
    m, k, n = 2, 50, 32
    w = torch.tensor([((i * 7 + 3) % 15) - 7.0 for i in range(n * k)], dtype=torch.float32).reshape(n, k)
    mw = rq.repack_marlin_tiles(w.to(dev), torch.full((n,), 0.5, device=dev))
    x = torch.tensor([np.sin(i * 0.1) for i in range(m * k)], dtype=torch.float32).reshape(1, m, k)
    y = rq.marlin_gemv(x.to(dev), mw)
    assert tuple(y.shape) == (1, m, n)
    deq = mw.dequantize()
    exp = x.reshape(m, k).to(dev) @ deq.t()
    assert torch.all((y.reshape(m, n) - exp).abs() < 1e-3)
    empty = rq.marlin_gemv(torch.zeros((0, k), device=dev), mw)
    assert tuple(empty.shape) == (0, n)


def test_linear_marlin_kats(dev):  # linear_layer.rs:143-185
    w = torch.tensor([[1.0, 2.0, 3.0, 4.0], [2.0, 3.0, 4.0, 5.0]], device=dev)
    mw = rq.repack_marlin_tiles(w, torch.ones(2, device=dev))
    assert mw.resident_bytes() == 2 * 4 * 4 + 2 * 4
    y = rq.marlin_gemv(torch.ones((1, 4), device=dev), mw)
    assert y.cpu().tolist() == [[10.0, 14.0]]
    with pytest.raises(rq.RqError):
        rq.marlin_gemv(torch.ones((1, 80), device=dev), mw)
    k, n = 64, 32
    w = torch.tensor([((i * 7 + 1) % 15) - 7.0 for i in range(n * k)]).reshape(n, k)
    mw = rq.repack_marlin_tiles(w.to(dev), torch.full((n,), 0.5, device=dev))
    x = torch.tensor([np.cos(i * 0.05) for i in range(k)], dtype=torch.float32).reshape(1, k).to(dev)
    y = rq.marlin_gemv(x, mw)
    exp = x @ mw.dequantize().t()
    assert torch.all((y - exp).abs() < 1e-3)


def test_errors(dev):  # MarlinWeight::new (marlin_gemv.rs:20-29)
    words = torch.zeros((1, 4, 4), dtype=torch.int32, device=dev)
    with pytest.raises(rq.RqError):
        rq.MarlinWeight(words, torch.ones(5, device=dev), 32, 4)     # scales not [out_dim]
    with pytest.raises(rq.RqError):
        rq.MarlinWeight(words, torch.ones(4, device=dev), 64, 4)     # needs 2 chunks of records
    with pytest.raises(rq.RqError):
        rq.MarlinWeight(words.float(), torch.ones(4, device=dev), 32, 4)  # packed not U32
    with pytest.raises(rq.RqError) as e:
        rq.check(rq.lib().rq_marlin_linear(None, None, 4, 32, None, rq.F32, 1, None, rq.F32, None))
    assert e.value.code == -5
