"""FP8 e4m3 path: activation encoders bit-exact against the oracle, the MFMA
GEMM against the f64 reference on the same quantized operands (gate 2e-2,
bf16 output), and the reference's own FP8 tests (fp8_gemm.rs:209-230,
fp8_weight.rs:135-157, linear_layer.rs:187-210) with their tolerances."""
import numpy as np
import pytest
import torch

import oracle
from runtimed_amd import rq, synth
from tests.conftest import norm_err

pytestmark = pytest.mark.gpu


def test_cuda_fp8_gemm_runs_or_skips(dev):  # fp8_gemm.rs:209-230
    m = n = k = 16
    x = torch.full((m, k), 0x38, dtype=torch.uint8, device=dev)
    w = torch.full((n, k), 0x38, dtype=torch.uint8, device=dev)
    s = torch.arange(1, 17, dtype=torch.float32, device=dev)
    y = rq.fp8_gemm(x.view(torch.float8_e4m3fn), w, s, out_dtype=torch.float32)
    assert y.shape == (m, n)
    ref = oracle.fp8_gemm_fallback(np.ones((m, k), np.float32), np.full((n, k), 0x38, np.uint8),
                                   s.cpu().numpy())
    assert np.all(np.abs(y.cpu().numpy() - ref) < 1e-1)


def test_fp8_weight_forward_matches_dequant(dev):  # fp8_weight.rs:135-157
    m = k = n = 16
    w = torch.full((n, k), 0x38, dtype=torch.uint8, device=dev)
    s = torch.arange(1, n + 1, dtype=torch.float32, device=dev) * 0.5
    x = torch.ones((m, k), dtype=torch.float32, device=dev)
    out = rq.fp8_gemm(x, w, s, mode=rq.FP8_UNSCALED, out_dtype=torch.float32).cpu().numpy()
    expected = np.ones((m, k), np.float32) @ (np.ones((n, k), np.float32) * s.cpu().numpy()[:, None]).T
    assert np.all(np.abs(out - expected) < 1e-1)


def test_linear_fp8_default_and_explicit_scale(dev):  # linear_layer.rs:187-210
    w = torch.full((16, 16), 0x38, dtype=torch.uint8, device=dev)
    x = torch.ones((1, 16), dtype=torch.float32, device=dev)
    y = rq.fp8_gemm(x, w, None, mode=rq.FP8_UNSCALED, out_dtype=torch.float32).cpu().numpy()
    assert y.shape == (1, 16) and np.all(np.abs(y - 16.0) < 1e-1)
    s = torch.arange(1, 17, dtype=torch.float32, device=dev)
    y = rq.fp8_gemm(x, w, s, mode=rq.FP8_UNSCALED, out_dtype=torch.float32).cpu().numpy()
    assert np.all(np.abs(y[0] - 16.0 * s.cpu().numpy()) < 1e-1)


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("k", [4096, 520, 72, 16384, 66])
def test_per_token_quantize_bit_exact(dev, xdt, k):
    # a wave per row from 16-byte loads where rows are 16-byte aligned (k = 66
    # is not: one workgroup per row, element loads)
    x = torch.from_numpy(synth.activations(11, 33, k) * 3.0).to(xdt)
    x[5] = 0.0
    x[7, 3] = float("nan")    # rows with NaN or infinity take the software encoder
    x[9, 1] = float("inf")
    x[11, 2] = -float("inf")
    xq, xs = rq.fp8_quantize(x.to(dev), rq.FP8_PER_TOKEN)
    want_q, want_s = oracle.fp8_quantize_rows(x.float().numpy())
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), want_s.view(np.uint32))
    assert np.array_equal(xq.cpu().numpy(), want_q)


def test_unscaled_encoder_bit_exact(dev):
    vals = np.concatenate([synth.normal(12, 50000) * 100.0, synth.normal(13, 5000) * 1e-3,
                           [0.0, -0.0, 448.0, 500.0, -1e9, np.inf, -np.inf, np.nan]]).astype(np.float32)
    t = torch.from_numpy(vals.reshape(1, -1)).to(dev)
    xq, xs = rq.fp8_quantize(t, rq.FP8_UNSCALED)
    assert np.array_equal(xq.cpu().numpy()[0], oracle.fp8_encode_array(vals))
    assert xs.cpu().numpy()[0] == 1.0


def test_unscaled_encoder_ties_and_boundaries(dev):
    # every e4m3 value, every midpoint between neighbours (exact ties, which
    # the reference breaks towards the lower magnitude) and the floats one ulp
    # either side of each, in both signs; the 2^-9 grid below 2^-6; values
    # around 448 and tiny or subnormal inputs
    pos = np.array([oracle.fp8_decode(c) for c in range(127)], np.float32)
    mids = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)
    assert np.array_equal(mids.astype(np.float64), (pos[:-1].astype(np.float64) + pos[1:]) / 2)
    near = np.concatenate([np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(np.inf)),
                           np.nextafter(pos, np.float32(0)), np.nextafter(pos, np.float32(np.inf))])
    grid = (np.arange(0, 8.01, 0.125, dtype=np.float32) / np.float32(512))
    extra = np.array([447.9, 448.0, 464.0, 479.9, 480.0, 1e-30, 1e-40, 2.0 ** -10, 2.0 ** -11, 3e-3],
                     np.float32)
    vals = np.concatenate([pos, mids, near, grid, extra]).astype(np.float32)
    vals = np.concatenate([vals, -vals])
    t = torch.from_numpy(vals.reshape(1, -1)).to(dev)
    xq, _ = rq.fp8_quantize(t, rq.FP8_UNSCALED)
    assert np.array_equal(xq.cpu().numpy()[0], oracle.fp8_encode_array(vals))


def _fp8_problem(m, n, k, seed):
    wv = synth.fp8_weight_values(seed, n, k)
    w = torch.from_numpy(wv).to("cuda")
    wq, _ = rq.fp8_quantize(w, rq.FP8_UNSCALED)   # the reference encoder, on the device
    ws = torch.from_numpy(synth.fp8_row_scales(seed, n)).to("cuda")
    xb = torch.from_numpy(synth.activations(seed + 1, m, k)).to(torch.bfloat16).to("cuda")
    return xb, wq, ws


@pytest.mark.parametrize("m,n,k", [(256, 512, 4096), (130, 200, 384), (1, 384, 256), (37, 1000, 128)])
def test_fp8_gemm_against_quantized_reference(dev, m, n, k):
    print(f"fp8 gemm m={m} n={n} k={k}", flush=True)
    xb, wq, ws = _fp8_problem(m, n, k, 90 + m)
    y = rq.fp8_gemm(xb, wq, ws, mode=rq.FP8_PER_TOKEN, out_dtype=torch.bfloat16).float().cpu().numpy()
    xq, xs = oracle.fp8_quantize_rows(xb.float().cpu().numpy())
    r = oracle.fp8_gemm_quantized_f64(xq, xs, wq.cpu().numpy(), ws.cpu().numpy())
    assert norm_err(y, r) <= 2e-2
    # f32 output on the same operands: only the summation differs from the f64
    # reference.  The fp8 matrix-core sum is measured at ~2e-5 normalized even
    # for k = 128 (its internal accumulation is not a plain f32 chain).
    y32 = rq.fp8_gemm(xb, wq, ws, out_dtype=torch.float32).cpu().numpy()
    assert norm_err(y32, r) <= 1e-4


def test_fp8_gemm_odd_k_scalar_path(dev):
    xb, wq, ws = _fp8_problem(9, 17, 96, 123)
    y = rq.fp8_gemm(xb, wq, ws, out_dtype=torch.float32).cpu().numpy()
    xq, xs = oracle.fp8_quantize_rows(xb.float().cpu().numpy())
    r = oracle.fp8_gemm_quantized_f64(xq, xs, wq.cpu().numpy(), ws.cpu().numpy())
    assert norm_err(y, r) <= 1e-5


def test_fp8_gemm_full_size_sampled(dev):
    # The 2048 x 14336 x 4096 workload, checked on sampled rows in f64.
    m, n, k = 2048, 14336, 4096
    xb, wq, ws = _fp8_problem(m, n, k, 7)
    y = rq.fp8_gemm(xb, wq, ws, out_dtype=torch.bfloat16)
    rows = np.array([0, 1, 777, 1500, 2047])
    xq, xs = oracle.fp8_quantize_rows(xb[rows].float().cpu().numpy())
    r = oracle.fp8_gemm_quantized_f64(xq, xs, wq.cpu().numpy(), ws.cpu().numpy())
    assert norm_err(y[rows].float().cpu().numpy(), r) <= 2e-2
    # information only: error against the reference's unquantized-x semantics
    ref_sem = oracle.fp8_gemm_fallback(xb[rows].float().cpu().numpy(), wq.cpu().numpy(), ws.cpu().numpy())
    print(f"per-token fp8 vs unquantized-x reference: {norm_err(y[rows].float().cpu().numpy(), ref_sem):.4f}")


@pytest.mark.parametrize("m,n,k", [(1300, 10000, 640), (513, 25700, 256), (1300, 10000, 1280), (2048, 14336, 192)])
def test_fp8_gemm_pipelined_ragged(dev, m, n, k):
    # >= 200 tiles of 256 x 256: the 4-stage direct-to-LDS kernels (eight
    # waves for k % 256 == 0, four otherwise), with ragged M/N edges and K-step
    # counts that are not a multiple of the stage count
    xb, wq, ws = _fp8_problem(m, n, k, 300 + m)
    y = rq.fp8_gemm(xb, wq, ws, out_dtype=torch.float32)
    rows = np.array([0, 1, m // 2, m - 2, m - 1])
    xq, xs = oracle.fp8_quantize_rows(xb[rows].float().cpu().numpy())
    r = oracle.fp8_gemm_quantized_f64(xq, xs, wq.cpu().numpy(), ws.cpu().numpy())
    assert norm_err(y[rows].cpu().numpy(), r) <= 1e-4
