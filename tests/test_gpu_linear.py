"""Fused quantized matmuls (rq_linear) against the dense reference
runtimed-gguf dequant + f32 matmul (linear_layer.rs:88-104), evaluated by the
oracle in double precision on the bit-exact dequantized weights.

Gate: normalized error max|y - r| / max|r| <= 1e-3 for f32 activations and
f32 accumulation (decode), <= 2e-2 where activations or outputs are bf16."""
import numpy as np
import pytest
import torch

import oracle
from runtimed_amd import rq, synth
from tests.conftest import norm_err

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3
TOL_BF16 = 2e-2


def make(qtype, n, k, seed):
    data = synth.weight_blocks(qtype, seed, n, k)
    rc, wf = oracle.dequant_tensor(qtype, data, n * k)
    assert rc == 0
    return rq.QWeight(qtype, data, n, k), wf.reshape(n, k)


def ref(x: np.ndarray, wf: np.ndarray) -> np.ndarray:
    return oracle.linear_f64(x, wf)


# The Q8_0 CPU-runnable workload (4864 x 896) and the Qwen2-0.5B decode set.
DECODE_SHAPES = [(4864, 896), (896, 896), (128, 896), (896, 4864)]


@pytest.mark.parametrize("qtype", [rq.Q8_0, rq.Q4_K, rq.Q6_K])
@pytest.mark.parametrize("n,k", DECODE_SHAPES + [(2048, 2048), (512, 8192), (96, 1024), (4100, 4096),
                                 (4096, 8192), (2048, 8192), (1601, 4864)])
def test_decode_gemv_f32(dev, qtype, n, k):
    # n >= 4096 with more than 64 pieces a row runs the one-wave-per-row kernel;
    # n < 4096 the team kernel, with four rows in flight where a workgroup
    # walks four or more (2048 x 8192; 1601 rows: workgroups of four and three)
    print(f"gemv qtype={qtype} n={n} k={k}", flush=True)
    w, wf = make(qtype, n, k, 10 + n + k)
    x = synth.activations(3, 1, k)
    y = w.forward(torch.from_numpy(x).to(dev)).cpu().numpy()
    assert y.shape == (1, n)
    assert norm_err(y, ref(x, wf)) <= TOL_F32


@pytest.mark.parametrize("qtype", [rq.Q4_K, rq.Q6_K, rq.Q8_0])
@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n,k", [(777, 4864), (1023, 2304), (513, 8192)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_two_team_gemv(dev, qtype, xdt, n, k, with_bias):
    # 512 < n <= 1024 rows of more than 64 pieces: two rows a workgroup, one
    # team each, x staged once in LDS; odd n leaves the last workgroup's second
    # row past the matrix (loaded clamped, never stored)
    w, wf = make(qtype, n, k, 71 + n + k)
    x = synth.activations(73 + n, 1, k)
    xt = torch.from_numpy(x).to(xdt)
    r = ref(xt.float().numpy(), wf)
    if with_bias:
        b = torch.from_numpy(synth.activations(75 + n, 1, n)[0]).to(dev)
        y = w.forward(xt.to(dev), out_dtype=torch.float32, bias=b).cpu().numpy()
        r = r + b.cpu().numpy()[None, :]
    else:
        y = w.forward(xt.to(dev), out_dtype=torch.float32).cpu().numpy()
    assert norm_err(y, r) <= TOL_F32


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n,k", [(4096, 512), (4096, 2048), (16394, 1024), (8192, 2048), (4133, 4096),
                                 (14336, 4096), (4096, 8192)])
def test_gemv_matrix_cores_q4k(dev, xdt, n, k):
    # M = 1 Q4_K with k % 512 == 0, k <= 8192 and n >= 4096 runs on the matrix
    # cores for k > 2048, and for k = 1024, 2048 where n k >= 2^24 (4096 x 512
    # and 4096 x 2048 stay on the segment kernel): the codes as bf16 128 + q,
    # x as two bf16 limbs (16 significant
    # bits), f32 sums; x spans six decades (N(0,1) with every 7th element
    # x300 and every 11th x1e-3), n = 4133 ends in a partial 32-row tile
    print(f"gemv mx x={xdt} n={n} k={k}", flush=True)
    w, wf = make(rq.Q4_K, n, k, 60 + n + k)
    x = synth.activations(5, 1, k)
    x[0, ::7] *= 300.0
    x[0, 3::11] *= 1e-3
    xt = torch.from_numpy(x).to(xdt)
    y = w.forward(xt.to(dev), out_dtype=torch.float32).cpu().numpy()
    assert y.shape == (1, n)
    assert norm_err(y, ref(xt.float().numpy(), wf)) <= TOL_F32


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n,k", [(14336, 4096), (65546, 1024), (32768, 2048), (16384, 4096), (8200, 8192)])
def test_gemv_matrix_cores_q6k(dev, xdt, n, k):
    # M = 1 Q6_K with k % 512 == 0, 1024 <= k <= 8192, n >= 4096 and
    # n k >= 2^26 runs on the matrix cores (14336 x 4096 just below the size
    # bound on the long-row kernel): 6-bit codes as bf16
    # 128 + q, one MFMA per 16-element sub-block with its int8 scale, x as two
    # bf16 limbs; x spans six decades, n = 65546 and 8200 end in a partial
    # 32-row tile
    print(f"gemv mx6 x={xdt} n={n} k={k}", flush=True)
    w, wf = make(rq.Q6_K, n, k, 61 + n + k)
    x = synth.activations(6, 1, k)
    x[0, ::7] *= 300.0
    x[0, 3::11] *= 1e-3
    xt = torch.from_numpy(x).to(xdt)
    y = w.forward(xt.to(dev), out_dtype=torch.float32).cpu().numpy()
    assert y.shape == (1, n)
    assert norm_err(y, ref(xt.float().numpy(), wf)) <= TOL_F32


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("qtype,n,k", [
    (rq.Q4_K, 4864, 896),   # 16-byte chunks of x per thread: 1 (f32) / 1 (16-bit)
    (rq.Q4_K, 512, 2048),   # 2 / 1
    (rq.Q6_K, 256, 4096),   # 4 / 2
    (rq.Q6_K, 128, 896),    # 1 / 1, Q6_K rows starting mid-block
    (rq.Q4_K, 896, 4864),   # three-wave teams, two rows per workgroup
    (rq.Q4_K, 64, 12288),   # six-wave teams
    (rq.Q8_0, 96, 16384),   # x too long for the LDS copy
    (rq.Q4_K, 1100, 20480),  # a ten-wave team, three rows per workgroup
    (rq.Q8_0, 4097, 8224),   # 257 pieces a row on n >= 4096: five-wave teams
])
def test_decode_gemv_activation_types(dev, xdt, qtype, n, k):
    # M = 1 with each activation type: x is read as raw 16-byte chunks (4 f32
    # or 8 f16/bf16 values) before the weights arrive, staged in LDS or, for
    # team layouts, held by the lanes that use it
    print(f"gemv x={xdt} qtype={qtype} n={n} k={k}", flush=True)
    w, wf = make(qtype, n, k, 20 + n + k)
    x = torch.from_numpy(synth.activations(4, 1, k)).to(xdt)
    y = w.forward(x.to(dev), out_dtype=torch.float32).cpu().numpy()
    assert y.shape == (1, n)
    # 16-bit activations are exact in f32: the f32 accumulation gate holds
    assert norm_err(y, ref(x.float().numpy(), wf)) <= TOL_F32


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("qtype,n,k", [(rq.Q4_K, 4864, 896), (rq.Q4_K, 130, 2048), (rq.Q6_K, 896, 896),
                                       (rq.Q8_0, 128, 896), (rq.Q5_K, 300, 512), (rq.Q4_0, 64, 2048),
                                       (rq.Q5_0, 77, 256),
                                       # long rows on fewer than 4096 rows: teams of 3, 4 and 10 waves
                                       (rq.Q4_K, 896, 4864), (rq.Q8_0, 300, 8192), (rq.Q4_0, 50, 20480)])
@pytest.mark.parametrize("m", [2, 3])
def test_few_rows_exact_weights(dev, xdt, qtype, n, k, m):
    # M = 2 runs the GEMVs with both activation rows (segment layout for rows
    # of at most 64 pieces, team layout for longer rows on n < 4096; Q6_K's
    # long rows excepted) for every activation type, M = 3 with f32 / f16
    # activations the segment layout with four row slots (rows of at most 64
    # pieces, Q6_K excepted): exact f32 weights and f32 accumulation, and
    # each row's result equal, bit for bit, to the M = 1 result of that row
    pieces = k // (64 if qtype == rq.Q6_K else 32)
    if m == 3 and (xdt == torch.bfloat16 or qtype == rq.Q6_K or pieces > 64):
        pytest.skip("three rows of this shape and type run on other kernels")
    print(f"few rows m={m} x={xdt} qtype={qtype} n={n} k={k}", flush=True)
    w, wf = make(qtype, n, k, 40 + n + k)
    x = torch.from_numpy(synth.activations(9 + m, m, k)).to(xdt).to(dev)
    y = w.forward(x, out_dtype=torch.float32)
    assert norm_err(y.cpu().numpy(), ref(x.float().cpu().numpy(), wf)) <= TOL_F32
    for i in range(m):
        y1 = w.forward(x[i:i + 1].contiguous(), out_dtype=torch.float32)
        assert torch.equal(y[i:i + 1], y1)


@pytest.mark.parametrize("n,k", [(896, 896), (128, 896), (896, 4864)])
@pytest.mark.parametrize("m", [2, 4, 8, 16, 64])
def test_verify_layer_shapes_bf16(dev, n, k, m):
    # The speculative-verify sweep on the other Qwen2-0.5B layer matrices
    # (q/o, k/v, down; gate/up is the case below): the small-M kernels run
    # them on 56 or 8 row tiles, unsplit (k = 896) or with K in slices
    # (down), with f32 and bf16 outputs
    print(f"verify layer n={n} k={k} m={m}", flush=True)
    w, wf = make(rq.Q4_K, n, k, 90 + n + m)
    xb = torch.from_numpy(synth.activations(91 + m, m, k)).to(torch.bfloat16)
    r = ref(xb.float().numpy(), wf)
    for ydt in (torch.float32, torch.bfloat16):
        y = w.forward(xb.to(dev), out_dtype=ydt).float().cpu().numpy()
        assert norm_err(y, r) <= TOL_BF16, (ydt, norm_err(y, r))


@pytest.mark.parametrize("qtype", [rq.Q4_K, rq.Q6_K, rq.Q8_0])
@pytest.mark.parametrize("m", [2, 4, 8, 16, 64])
def test_verify_small_m_bf16(dev, qtype, m):
    n, k = 896, 4864
    if qtype == rq.Q4_K:
        n, k = 4864, 896
    print(f"verify qtype={qtype} m={m}", flush=True)
    w, wf = make(qtype, n, k, 20 + m)
    xb = torch.from_numpy(synth.activations(4 + m, m, k)).to(torch.bfloat16)
    y = w.forward(xb.to(dev), out_dtype=torch.float32).cpu().numpy()
    assert norm_err(y, ref(xb.float().numpy(), wf)) <= TOL_BF16


# The small-M matrix-core kernel (2 <= m <= 64): partial column tiles
# (m = 3, 17, 33, 63), weight rows not a multiple of 16, fewer K-chunks than
# waves (k = 64, 128), rows straddling super-blocks (k = 896), long K in
# several batches a wave (k = 1088, 4864, 8192), and bf16 / f16 outputs.
# From 16 rows with k <= 2048 the activation slice is copied to LDS: in
# several rounds of the copy (64 x 2048), with K split over workgroups
# (256 rows: 16 row tiles, eight slices) and unsplit (2048 rows).
@pytest.mark.parametrize("qtype", [rq.Q4_K, rq.Q6_K, rq.Q8_0])
@pytest.mark.parametrize("m,n,k", [(3, 37, 256), (17, 130, 128), (33, 100, 896), (63, 200, 64), (5, 4864, 896),
                                   (3, 130, 4864), (33, 40, 8192), (17, 96, 1088), (64, 256, 2048),
                                   (16, 2048, 2048), (40, 2048, 1024)])
def test_small_m_edges(dev, qtype, m, n, k):
    w, wf = make(qtype, n, k, 31 + m + n)
    xb = torch.from_numpy(synth.activations(6 + m, m, k)).to(torch.bfloat16)
    r = ref(xb.float().numpy(), wf)
    for ydt in (torch.float32, torch.bfloat16, torch.float16):
        y = w.forward(xb.to(dev), out_dtype=ydt).float().cpu().numpy()
        assert norm_err(y, r) <= TOL_BF16, (ydt, norm_err(y, r))


@pytest.mark.parametrize("qtype", [rq.Q4_K, rq.Q6_K])
def test_prefill_bf16_out(dev, qtype):
    m, n, k = 128, 1024, 2048
    w, wf = make(qtype, n, k, 31)
    xb = torch.from_numpy(synth.activations(5, m, k)).to(torch.bfloat16)
    y = w.forward(xb.to(dev)).float().cpu().numpy()
    assert norm_err(y, ref(xb.float().numpy(), wf)) <= TOL_BF16


# f32 and f16 activations with 4 <= M <= 64 run on the f32 matrix cores
# (v_mfma_f32_16x16x4_f32) with the exact dequantized weights: the f32
# tolerance holds; M < 4, M > 64 and K % 64 != 0 stay on the VALU kernel.
# The 0.5B layer's gate / q shapes at 16 and 32 rows, and 16 x 1536 (more
# than one batch a wave: sixteen waves).
ALL_FORMATS = [rq.Q4_K, rq.Q6_K, rq.Q8_0, rq.Q5_K, rq.Q4_0, rq.Q5_0]


@pytest.mark.parametrize("qtype", ALL_FORMATS)
@pytest.mark.parametrize("m,n,k", [(2, 4864, 896), (4, 4864, 896), (5, 130, 256), (16, 896, 4864), (17, 300, 512),
                                   (40, 64, 2048), (64, 258, 128), (65, 96, 256), (16, 4864, 896), (32, 896, 896),
                                   (16, 300, 1536)])
def test_small_m_f32_activations(dev, qtype, m, n, k):
    w, wf = make(qtype, n, k, 17 + m + n)
    x = torch.from_numpy(synth.activations(5 + m, m, k))
    y = w.forward(x.to(dev)).cpu().numpy()
    assert y.dtype == np.float32
    assert norm_err(y, ref(x.numpy(), wf)) <= TOL_F32


# f32 activations with 4 <= M <= 16 on Q4_K / Q6_K / Q8_0 (17..32 rows on rows
# longer than 2048, on 256 or more row tiles and in sets; 33..64 rows on 256 or
# more row tiles: 40 x 4100, 64 x 4864; 20 x 300 only as the set below) take
# the integer codes on the bf16 matrix cores (128 + q,
# or the int8 code, exact in bf16) against two bf16 limbs of x, the scales
# applied per run of 16 or 32 weights to the f32 sums.  x spans six decades
# (every 7th element x300, every 11th x1e-3); launches of 256 or more row
# tiles take two a workgroup (4864 rows, and 4100 = 256.25 tiles: a last
# workgroup with one); few row tiles on long rows split
# K over up to four workgroups (7 x 4096, 16 x 4096, 24 x 8192), the
# activation slice is staged in LDS (16 x 896, 16 x 4096 in four slices,
# 17 x 4864) or read from memory (m < 16, 16 x 8192, 31 x 4096), rows straddle
# blocks (k = 896 for the 256-element formats), and m, n end in partial tiles.
@pytest.mark.parametrize("qtype", [rq.Q4_K, rq.Q6_K, rq.Q8_0])
@pytest.mark.parametrize("m,n,k", [(4, 4864, 896), (7, 100, 4096), (16, 896, 896), (16, 64, 4096),
                                   (16, 64, 8192), (17, 896, 4864), (31, 200, 4096), (24, 40, 8192),
                                   (31, 4100, 4096), (20, 300, 896), (40, 4100, 1024), (64, 4864, 896)])
def test_small_m_f32_codes(dev, qtype, m, n, k):
    print(f"codes qtype={qtype} m={m} n={n} k={k}", flush=True)
    w, wf = make(qtype, n, k, 41 + m + n + k)
    x = synth.activations(9 + m, m, k)
    x[:, ::7] *= 300.0
    x[:, 3::11] *= 1e-3
    r = ref(x, wf)
    y = w.forward(torch.from_numpy(x).to(dev)).cpu().numpy()
    assert norm_err(y, r) <= TOL_F32
    # per row as well: a row of small activations is not hidden by the others
    for i in range(m):
        assert norm_err(y[i:i + 1], r[i:i + 1]) <= TOL_F32, i
    # a set of three weights of the format sharing x, each as its own call
    others = [make(qtype, nn, k, 43 + nn + i) for i, nn in enumerate((n, 16, 34))]
    xt = torch.from_numpy(x).to(dev)
    outs = rq.linear_multi([o for o, _ in others], xt, out_dtype=torch.float32)
    for (o, of), yo in zip(others, outs):
        assert norm_err(yo.cpu().numpy(), ref(x, of)) <= TOL_F32
        assert norm_err(yo.cpu().numpy(), o.forward(xt).cpu().numpy()) <= 1e-5


# More than 64 f32 rows run on the tiled GEMM with two bf16 limbs per
# operand (exact weights split into hi + lo, f32 accumulation): tiles past
# m and n, rows straddling Q4_K blocks (k = 896), k not a multiple of 128
# (640), and 64 x 64 / 128 x 128 tiles all occur here.
@pytest.mark.parametrize("qtype", [rq.Q4_K, rq.Q6_K, rq.Q8_0, rq.Q5_0])
@pytest.mark.parametrize("m,n,k", [(200, 300, 512), (129, 130, 256), (66, 64, 2048), (131, 96, 896),
                                   (512, 1000, 1024), (300, 2048, 640)])
def test_f32_activations_sliced(dev, qtype, m, n, k):
    w, wf = make(qtype, n, k, 23 + m)
    x = torch.from_numpy(synth.activations(7 + m, m, k))
    for ydt in (torch.float32, torch.bfloat16):
        y = w.forward(x.to(dev), out_dtype=ydt).float().cpu().numpy()
        tol = TOL_F32 if ydt == torch.float32 else TOL_BF16
        assert norm_err(y, ref(x.numpy(), wf)) <= tol


# f32 activations with m > 64 on the two-limb tiles, row by row: rows of very
# different magnitudes (1e-30, 1e-3, 1e20), a row of zeros, x spanning six
# decades inside rows; 64 x 64 tiles in K-groups (k = 2048, 896, 256),
# 128 x 128 tiles (512 x 4096) and K split four ways (k = 8192).
@pytest.mark.parametrize("m,n,k", [(96, 512, 2048), (200, 300, 896), (130, 2048, 8192), (65, 8192, 256),
                                   (512, 4096, 512)])
def test_f32_prefill_row_magnitudes(dev, m, n, k):
    print(f"f32 prefill rows m={m} n={n} k={k}", flush=True)
    w, wf = make(rq.Q4_K, n, k, 61 + m)
    x = synth.activations(62 + m, m, k)
    x[:, ::7] *= 300.0
    x[:, 3::11] *= 1e-3
    x[1] *= 1e-30
    x[2] *= 1e20
    x[3] = 0.0
    x[4] *= 1e-3
    r = ref(x, wf)
    y = w.forward(torch.from_numpy(x).to(dev)).cpu().numpy()
    assert np.all(y[3] == 0.0)
    for i in [i for i in range(m) if i != 3]:
        assert norm_err(y[i:i + 1], r[i:i + 1]) <= TOL_F32, i


@pytest.mark.parametrize("qtype", [rq.Q4_K, rq.Q6_K, rq.Q8_0])
@pytest.mark.parametrize("m", [3, 33])
def test_small_m_f16_activations(dev, qtype, m):
    w, wf = make(qtype, 200, 896, 3 + m)
    x = torch.from_numpy(synth.activations(8 + m, m, 896)).to(torch.float16)
    y = w.forward(x.to(dev), out_dtype=torch.float32).cpu().numpy()
    # f16 activations are exact in f32; f32 accumulation
    assert norm_err(y, ref(x.float().numpy(), wf)) <= TOL_F32


@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float16), (torch.float16, torch.float32),
                                     (torch.bfloat16, torch.bfloat16)])
def test_activation_and_output_types(dev, xdt, ydt):
    w, wf = make(rq.Q4_K, 256, 512, 41)
    x = torch.from_numpy(synth.activations(6, 3, 512)).to(xdt)
    y = w.forward(x.to(dev), out_dtype=ydt).float().cpu().numpy()
    tol = TOL_F32 if (xdt == torch.float32 and ydt == torch.float32) else TOL_BF16
    assert norm_err(y, ref(x.float().numpy(), wf)) <= tol


@pytest.mark.parametrize("qtype,n,k", [
    (rq.Q4_K, 8, 160),    # k % 64 != 0: rows cut inside a chunk -> decode path
    (rq.Q8_0, 2, 48),     # k % 32 != 0: blocks straddle rows mid-block
    (rq.Q6_K, 2, 384),    # fused, row 1 starts in the second half of block 1
    (rq.Q6_K, 4, 192),    # k % 128 != 0 -> decode path
    (rq.Q4_0, 64, 96), (rq.Q5_0, 64, 96), (rq.Q5_K, 32, 512),
])
def test_other_shapes_and_formats(dev, qtype, n, k):
    w, wf = make(qtype, n, k, 51 + k)
    for m in (1, 5):
        x = synth.activations(7 + m, m, k)
        y = w.forward(torch.from_numpy(x).to(dev)).cpu().numpy()
        assert norm_err(y, ref(x, wf)) <= TOL_F32


def test_k896_rows_straddle_blocks(dev):
    # K = 896 puts 3.5 super-blocks in a row: odd rows start mid-block.  A
    # single nonzero input column isolates W[:, j] exactly.
    n, k = 6, 896
    w, wf = make(rq.Q4_K, n, k, 61)
    for j in (0, 127, 128, 255, 640, 767, 768, 895):
        x = np.zeros((1, k), np.float32)
        x[0, j] = 1.0
        y = w.forward(torch.from_numpy(x).to(dev)).cpu().numpy()[0]
        assert np.array_equal(y, wf[:, j])


def test_zero_rows_is_noop(dev):
    w, _ = make(rq.Q4_K, 64, 256, 71)
    x = torch.empty((0, 256), device=dev)
    assert w.forward(x).shape == (0, 64)


def test_linear_dense_and_quantized_kat(dev):
    # linear_layer.rs:129-140 and the Marlin KAT [10, 14] of linear_layer.rs:143-155,
    # here with Q8_0 blocks holding the small integer weights exactly (d = 1).
    rows = [[1, 2, 3, 4] + [0] * 28, [2, 3, 4, 5] + [0] * 28]
    blocks = b"".join(bytes([0x00, 0x3C]) + bytes(np.array(r, np.int8).view(np.uint8)) for r in rows)
    w = rq.QWeight(rq.Q8_0, np.frombuffer(blocks, np.uint8), 2, 32)
    x = torch.zeros((1, 32), device=dev)
    x[0, :4] = 1.0
    y = w.forward(x).cpu().numpy()
    assert y.shape == (1, 2) and y[0].tolist() == [10.0, 14.0]


def test_golden_gemv_on_device(dev):
    from tests.golden import load_golden

    for case in load_golden()["gemv"]:
        w = rq.QWeight(case["qtype"], case["blocks"], case["n"], case["k"])
        y = w.forward(torch.from_numpy(case["x"]).to(dev)).cpu().numpy()
        assert norm_err(y, case["y"]) <= TOL_F32, case["name"]


@pytest.mark.parametrize("qtype", [rq.Q4_K, rq.Q6_K, rq.Q8_0])
@pytest.mark.parametrize("m,n,k", [(257, 130, 512), (33, 1000, 256), (65, 64, 1024), (300, 256, 2048),
                                   (300, 256, 8192), (129, 200, 8384), (300, 128, 448), (300, 16384, 640),
                                   (257, 8192, 2048), (300, 16384, 576)])
def test_mfma_gemm_edge_tiles(dev, qtype, m, n, k):
    # K >= 4096 with few tiles splits K across workgroups (f32 partials, then
    # a sum); 8384 = 131 K-steps leaves a shorter last split.  Inside a
    # workgroup K is split over groups of waves: four on 64 x 64 tiles (k =
    # 512, 1024, 2048: 2, 4 and 8 steps a group), two on 128 x 128 tiles
    # (k = 640 and 2048: 5 and 16 steps a group); 448 (7 steps) and 576
    # (9 steps) do not divide and run one group.
    # bf16 activations with m > 1 run on the matrix cores; tiles are 32..256 x 128
    w, wf = make(qtype, n, k, 81 + m + n)
    xb = torch.from_numpy(synth.activations(9 + m, m, k)).to(torch.bfloat16)
    for ydt in (torch.float32, torch.bfloat16):
        y = w.forward(xb.to(dev), out_dtype=ydt).float().cpu().numpy()
        assert norm_err(y, ref(xb.float().numpy(), wf)) <= TOL_BF16


# Shapes with >= 256 tiles of 256 x 256 run the 256 x 256 tile kernel:
# exact tiles, ragged rows and columns, rows that straddle super-blocks
# (k % 256 != 0), odd and single K-step counts.
@pytest.mark.parametrize("qtype,m,n,k", [
    (rq.Q4_K, 512, 32768, 256),
    (rq.Q6_K, 300, 32868, 320),
    (rq.Q8_0, 257, 33000, 128),
    (rq.Q4_K, 512, 32768, 64),
    (rq.Q6_K, 512, 32768, 448),
    (rq.Q6_K, 768, 32768, 256),  # pipelined kernel, three M tiles per weight tile in the XCD-aware order
    (rq.Q6_K, 300, 32868, 512),  # pipelined Q6_K, ragged rows and columns (accumulator stores)
    (rq.Q6_K, 512, 32776, 1024),  # pipelined Q6_K, ragged last column tile, whole tiles staged
    (rq.Q6_K, 300, 32868, 384),  # Q6_K with k % 256 != 0: the per-chunk pipelined kernel, ragged
    (rq.Q8_0, 512, 32768, 640),  # pipelined, whole tiles staged
    (rq.Q6_K, 100, 65600, 512),  # pipelined Q6_K, one M tile of 100 rows
    (rq.Q4_K, 100, 65600, 384),  # pipelined, one M tile of 100 rows
])
def test_large_gemm(dev, qtype, m, n, k):
    w, wf = make(qtype, n, k, 5 + m + k)
    xb = torch.from_numpy(synth.activations(3 + m, m, k)).to(torch.bfloat16)
    r = oracle.linear_f32(xb.float().numpy(), wf, threads=8)
    for ydt in (torch.bfloat16, torch.float32):
        y = w.forward(xb.to(dev), out_dtype=ydt).float().cpu().numpy()
        assert norm_err(y, r) <= TOL_BF16, (ydt, norm_err(y, r))


# Q5_K, Q4_0 and Q5_0 on the fused paths: M = 1 (VALU GEMV, f32 gate),
# small M and the tiled GEMM (bf16 gate); Q4_0 / Q5_0 are uploaded in split
# layouts (16 quant bytes per block, then d / {qh, d} records).
NEXT_FORMATS = [rq.Q5_K, rq.Q4_0, rq.Q5_0]


@pytest.mark.parametrize("qtype", NEXT_FORMATS)
@pytest.mark.parametrize("n,k", [(4864, 896), (896, 4864), (130, 256), (64, 2048)])
def test_next_formats_gemv_f32(dev, qtype, n, k):
    w, wf = make(qtype, n, k, 41 + n)
    x = synth.activations(43, 1, k)
    y = w.forward(torch.from_numpy(x).to(dev)).cpu().numpy()
    assert norm_err(y, ref(x, wf)) <= TOL_F32


@pytest.mark.parametrize("qtype", NEXT_FORMATS)
@pytest.mark.parametrize("m,n,k", [(2, 896, 896), (17, 130, 256), (64, 200, 1024), (300, 256, 2048),
                                   (512, 1024, 512), (300, 32868, 256)])
def test_next_formats_matrix_cores(dev, qtype, m, n, k):
    w, wf = make(qtype, n, k, 47 + m)
    xb = torch.from_numpy(synth.activations(49 + m, m, k)).to(torch.bfloat16)
    r = ref(xb.float().numpy(), wf)
    for ydt in (torch.float32, torch.bfloat16):
        y = w.forward(xb.to(dev), out_dtype=ydt).float().cpu().numpy()
        assert norm_err(y, r) <= TOL_BF16, (ydt, norm_err(y, r))


@pytest.mark.parametrize("qtype", NEXT_FORMATS + [rq.Q8_0])
@pytest.mark.parametrize("m,n,k", [(130, 256, 2048), (300, 2048, 4096), (512, 4096, 512)])
def test_next_formats_f32_prefill(dev, qtype, m, n, k):
    # f32 activations above 64 rows: the two-limb tiles (64 x 64 in four
    # single-buffered K-groups, 128 x 128 in two, split K for long rows; Q8_0
    # and Q5_0 keep double-buffered groups where the wide form would spill)
    w, wf = make(qtype, n, k, 53 + m)
    x = synth.activations(55 + m, m, k)
    y = w.forward(torch.from_numpy(x).to(dev)).cpu().numpy()
    assert norm_err(y, ref(x, wf)) <= TOL_F32


@pytest.mark.parametrize("qtype", [rq.Q4_K, rq.Q8_0, rq.Q6_K])
def test_fused_weights_concatenate(dev, qtype):
    # q/k/v (and gate/up) each hold a whole number of blocks, so their GGUF
    # streams concatenate into one weight whose rows are the stacked rows;
    # each output row is computed the same way, so the results are identical.
    parts = [(896, 896), (128, 896), (128, 896)]
    data = [synth.weight_blocks(qtype, 300 + i, n, 896) for i, (n, _) in enumerate(parts)]
    x = torch.from_numpy(synth.activations(9, 1, 896)).to(dev)
    sep = [rq.QWeight(qtype, d, n, 896).forward(x) for d, (n, _) in zip(data, parts)]
    fused = rq.QWeight(qtype, np.concatenate(data), 1152, 896).forward(x)
    assert torch.equal(fused, torch.cat(sep, dim=1))


def _random_cases(count=48, seed=2024):
    """Seeded shapes across every format, activation type and row count: rows
    that straddle blocks, n not a multiple of any tile, k from one block to a
    few thousand, M from the GEMV through the small-M kernels to the tiled
    GEMM and the f32 slices."""
    rng = np.random.default_rng(seed)
    ks = [32, 64, 96, 160, 256, 384, 896, 1024, 1088, 2048, 2304, 4864, 5120]
    ms = [1, 1, 1, 2, 3, 4, 7, 16, 17, 33, 64, 65, 130]
    xts = [torch.float32, torch.float16, torch.bfloat16]
    out = []
    while len(out) < count:
        qt = ALL_FORMATS[rng.integers(len(ALL_FORMATS))]
        k = int(ks[rng.integers(len(ks))])
        elems = rq.GEOMETRY[qt][0]
        n = int(rng.integers(1, 3000))
        while (n * k) % elems:
            n += 1
        if n * k > 6_000_000:
            continue
        out.append((qt, n, k, int(ms[rng.integers(len(ms))]), xts[rng.integers(len(xts))]))
    return out


@pytest.mark.parametrize("qtype,n,k,m,xdt", _random_cases())
def test_random_shapes(dev, qtype, n, k, m, xdt):
    print(f"random qtype={qtype} n={n} k={k} m={m} x={xdt}", flush=True)
    w, wf = make(qtype, n, k, 7 * n + k + m)
    x = torch.from_numpy(synth.activations(n + m, m, k)).to(xdt)
    y = w.forward(x.to(dev), out_dtype=torch.float32).cpu().numpy()
    assert y.shape == (m, n)
    # bf16 activations with m > 1 run on bf16 matrix cores (weights rounded to
    # bf16); every other case keeps exact weights and f32 accumulation
    tol = TOL_BF16 if (xdt == torch.bfloat16 and m > 1) else TOL_F32
    assert norm_err(y, ref(x.float().numpy(), wf)) <= tol
