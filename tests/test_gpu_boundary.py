"""The linear boundary beyond y = x W^T: linear_bias's bias (linear_layer.rs:
107-118) in every kernel's epilogue, the last-dimension check of
linear_layer.rs:88-96, activations at any alignment, several linears on one
input in one launch (qwen2.rs:99-125 calls q/k/v and gate/up that way),
shapes no fused kernel takes, and the per-stream workspace under graph
capture.

Reference: runtimed-gguf dequant + dense matmul evaluated by the oracle in
f64, plus the bias.  Gates: normalized error <= 1e-3 with f32 activations and
outputs, <= 2e-2 with bf16 operands; bit-exact where the same kernels run."""
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


def bias_vec(n, seed, dtype, dev):
    return torch.from_numpy(synth.activations(seed, 1, n)[0]).to(dtype).to(dev)


# Every kernel family of the fused path: segment / team / long-row /
# matrix-core GEMVs (M = 1, 2), the small-M matrix-core kernels (bf16 and f32), the tiled GEMM
# with and without split K, the pipelined 256 x 256 kernels, the f32 slices,
# and the generic kernel (k % 64 != 0).
ROUTES = [
    # (qtype, n, k, m, xdtype)
    (rq.Q4_K, 4864, 896, 1, torch.float32),     # segment GEMV
    (rq.Q4_K, 896, 4864, 1, torch.float32),     # team GEMV
    (rq.Q4_K, 4100, 4096, 1, torch.float32),    # matrix-core GEMV (Q4_K long rows)
    (rq.Q4_K, 8200, 2048, 1, torch.float16),    # matrix-core GEMV (Q4_K 64-piece rows, n k >= 2^24)
    (rq.Q6_K, 32800, 2048, 1, torch.bfloat16),  # matrix-core GEMV (Q6_K, n k >= 2^26)
    (rq.Q8_0, 4100, 4096, 1, torch.float32),    # one wave per row
    (rq.Q6_K, 896, 896, 2, torch.float32),      # two rows, segment
    (rq.Q4_K, 896, 4864, 2, torch.bfloat16),    # two rows, team
    (rq.Q8_0, 128, 896, 16, torch.bfloat16),    # small-M bf16 MFMA
    (rq.Q4_K, 300, 2048, 16, torch.float32),    # small-M f32 MFMA
    (rq.Q4_K, 1024, 2048, 300, torch.bfloat16),  # tiled GEMM
    (rq.Q6_K, 256, 8192, 300, torch.bfloat16),  # split K
    (rq.Q4_K, 32768, 256, 512, torch.bfloat16),  # pipelined 256 x 256
    (rq.Q6_K, 32768, 256, 512, torch.bfloat16),  # pipelined 256 x 256, eight waves (Q6_K chunk pairs)
    (rq.Q8_0, 130, 256, 131, torch.float32),    # f32 slices with a 3-row tail
    (rq.Q4_K, 8, 160, 5, torch.float32),        # generic (rows cut mid-chunk)
]


@pytest.mark.parametrize("qtype,n,k,m,xdt", ROUTES)
@pytest.mark.parametrize("bdt", [torch.float32, torch.float16, torch.bfloat16])
def test_linear_bias_every_route(dev, qtype, n, k, m, xdt, bdt):
    print(f"bias qtype={qtype} n={n} k={k} m={m} x={xdt} b={bdt}", flush=True)
    w, wf = make(qtype, n, k, 600 + n + m)
    x = torch.from_numpy(synth.activations(601 + m, m, k)).to(xdt).to(dev)
    b = bias_vec(n, 602 + n, bdt, dev)
    b64 = b.double().cpu().numpy()
    r = oracle.linear_f64(x.float().cpu().numpy(), wf) + b64[None, :]
    # exact f32 weights and accumulation except bf16 activations beyond two
    # rows (bf16 matrix cores)
    exact = xdt != torch.bfloat16 or m <= 2
    for ydt in (torch.float32, torch.bfloat16):
        y = w.forward(x, out_dtype=ydt, bias=b)
        tol = TOL_F32 if exact and ydt == torch.float32 else TOL_BF16
        err = norm_err(y.float().cpu().numpy(), r)
        assert err <= tol, (ydt, err)
        # against linear then the broadcast add (linear_layer.rs:107-118: y
        # rounded to its dtype, the bias cast to it, the sum rounded again):
        # the fused epilogue makes the same two roundings, bit for bit
        y0 = w.forward(x, out_dtype=ydt)
        rq.bias_add(y0, b)
        assert torch.equal(y, y0), ydt


def test_bias_add_semantics(dev):
    # linear_layer.rs:111-115: the bias is cast to y's dtype, then added
    y = torch.tensor([[1.0, 2.0], [3.0, 4.0]], dtype=torch.bfloat16, device=dev)
    b = torch.tensor([0.5, 1.0 + 2.0 ** -10], dtype=torch.float32, device=dev)  # rounds to 1.0 in bf16
    rq.bias_add(y, b)
    assert y.float().cpu().tolist() == [[1.5, 3.0], [3.5, 5.0]]
    y32 = torch.zeros((3, 2), device=dev)
    rq.bias_add(y32, b)
    assert torch.equal(y32.cpu(), b.cpu().expand(3, 2))


def test_wrong_width_is_a_shape_error(dev):
    # linear_layer.rs:88-96: a last dimension other than the weight's k is
    # ModelError::Shape, and nothing is launched
    w, _ = make(rq.Q4_K, 64, 512, 3)
    for bad in (256, 511, 513, 1024):
        x = torch.zeros((2, bad), device=dev)
        y = torch.full((2, 64), 7.0, device=dev)
        with pytest.raises(rq.RqError) as e:
            w.forward(x, out=y)
        assert e.value.kind == "Shape" and "expected last dim 512" in e.value.message
        assert bool(torch.all(y == 7.0))
    with pytest.raises(rq.RqError) as e:
        rq.linear_multi([w, w], torch.zeros((1, 256), device=dev))
    assert e.value.kind == "Shape"


def _offset_view(x: torch.Tensor, elems: int) -> torch.Tensor:
    """x's values in a contiguous tensor whose data starts `elems` elements
    past a 256-byte boundary."""
    buf = torch.empty(x.numel() + 64, dtype=x.dtype, device=x.device)
    v = buf[elems:elems + x.numel()].view(x.shape)
    v.copy_(x)
    assert v.data_ptr() % 16 == (elems * x.element_size()) % 16
    return v


def test_unaligned_activations_lm_head(dev):
    # The Q6_K 262144 x 2048 output projection with bf16 activations starting
    # 2, 4 and 6 bytes past an aligned address: x is copied (m * k elements)
    # into the stream's workspace and runs on the same kernel, so the result
    # equals the aligned call's bit for bit.
    n, k, m = 262144, 2048, 512
    print(f"unaligned head n={n} k={k} m={m}", flush=True)
    data = synth.weight_blocks(rq.Q6_K, 77, n, k)
    w = rq.QWeight(rq.Q6_K, data, n, k)
    x = torch.from_numpy(synth.activations(78, m, k)).to(torch.bfloat16).to(dev)
    y_ref = w.forward(x, out_dtype=torch.float32)
    cols = np.arange(0, n, 257)
    rows_bytes = []
    per_row = k // 256 * 210
    for c in cols:
        rows_bytes.append(data[c * per_row:(c + 1) * per_row])
    rc, wf = oracle.dequant_tensor(rq.Q6_K, np.concatenate(rows_bytes), len(cols) * k, threads=8)
    assert rc == 0
    r = oracle.linear_f64(x.float().cpu().numpy(), wf.reshape(len(cols), k))
    assert norm_err(y_ref[:, torch.from_numpy(cols).to(dev)].cpu().numpy(), r) <= TOL_BF16
    for off in (1, 2, 3):
        xv = _offset_view(x, off)
        y = w.forward(xv, out_dtype=torch.float32)
        assert torch.equal(y, y_ref), off
    # f32 activations 4 bytes past alignment, M = 1
    x1 = torch.from_numpy(synth.activations(79, 1, k)).to(dev)
    assert torch.equal(w.forward(_offset_view(x1, 1)), w.forward(x1))
    w.close()


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 2, 3, 16, 33, 64])
def test_linear_multi_matches_separate_calls(dev, xdt, m):
    # q/k/v (Q4_K 896 / 128 / 128 x 896) with biases, then gate/up: one
    # launch per set, each output identical to its own rq_linear_bias call
    # and within the gate of the oracle (dequant + f64 matmul + bias)
    print(f"multi m={m} x={xdt}", flush=True)
    k = 896
    tol = TOL_F32 if xdt == torch.float32 else TOL_BF16
    # bf16 activations beyond two rows and f32 ones beyond three run as one
    # small-M set launch, which may split K over a different number of
    # workgroups than a single weight, so only the summation order differs
    # (within f32 rounding); otherwise the same kernels run
    exact = not ((xdt == torch.bfloat16 and m >= 3) or (xdt == torch.float32 and m >= 4))

    def same(a, b):
        if exact:
            return torch.equal(a, b)
        return norm_err(a.cpu().numpy(), b.cpu().numpy()) <= 1e-5

    def oracle_ok(y, wf, xin, b=None):
        r = oracle.linear_f64(xin.float().cpu().numpy(), wf)
        if b is not None:
            r = r + b.float().cpu().numpy().astype(np.float64)
        return norm_err(y.cpu().numpy(), r) <= tol
    made = [make(rq.Q4_K, n, k, 700 + i) for i, n in enumerate((896, 128, 128))]
    ws = [w for w, _ in made]
    x = torch.from_numpy(synth.activations(710 + m, m, k)).to(xdt).to(dev)
    bs = [bias_vec(w.n, 720 + i, torch.float16, dev) for i, w in enumerate(ws)]
    outs = rq.linear_multi(ws, x, biases=bs, out_dtype=torch.float32)
    for (w, wf), b, y in zip(made, bs, outs):
        assert same(y, w.forward(x, out_dtype=torch.float32, bias=b))
        assert oracle_ok(y, wf, x, b)
    # bf16 outputs with biases: the set's epilogue rounds the product, adds
    # the rounded bias and rounds again, as the set without biases followed
    # by the broadcast add does (linear_layer.rs:107-118), bit for bit
    outs16 = rq.linear_multi(ws, x, biases=bs, out_dtype=torch.bfloat16)
    plain16 = rq.linear_multi(ws, x, out_dtype=torch.bfloat16)
    for b, y, y0 in zip(bs, outs16, plain16):
        rq.bias_add(y0, b)
        assert torch.equal(y, y0)
    gu_made = [make(rq.Q4_K, 4864, k, 730 + i) for i in range(2)]
    gu = [w for w, _ in gu_made]
    outs = rq.linear_multi(gu, x, out_dtype=torch.float32)
    for (w, wf), y in zip(gu_made, outs):
        assert same(y, w.forward(x, out_dtype=torch.float32))
        assert oracle_ok(y, wf, x)
    assert all(torch.equal(a, b) for a, b in zip(outs, rq.linear_multi(gu, x, out_dtype=torch.float32)))
    # a mixed set (Q4_K, Q4_K, Q6_K as Q4_K_M stores q / k / v) and a set
    # with long rows: grouped by format, each output as its own call
    mixed_made = [make(rq.Q4_K, 896, k, 740), make(rq.Q4_K, 128, k, 741), make(rq.Q6_K, 128, k, 742)]
    mixed = [w for w, _ in mixed_made]
    mixed_bias = [None, bs[1], None]
    for (w, wf), b, y in zip(mixed_made, mixed_bias, rq.linear_multi(mixed, x, biases=mixed_bias,
                                                                     out_dtype=torch.float32)):
        assert same(y, w.forward(x, out_dtype=torch.float32, bias=b))
        assert oracle_ok(y, wf, x, b)
    longs_made = [make(rq.Q4_K, 896, 4864, 750), make(rq.Q4_K, 300, 4864, 751)]
    x2 = torch.from_numpy(synth.activations(752, m, 4864)).to(xdt).to(dev)
    for (w, wf), y in zip(longs_made, rq.linear_multi([w for w, _ in longs_made], x2, out_dtype=torch.float32)):
        assert same(y, w.forward(x2, out_dtype=torch.float32))
        assert oracle_ok(y, wf, x2)


def test_linear_multi_against_oracle(dev):
    k = 896
    shapes = [(896, rq.Q4_K), (128, rq.Q4_K), (128, rq.Q4_K), (4864, rq.Q4_K)]
    made = [make(qt, n, k, 760 + i) for i, (n, qt) in enumerate(shapes)]
    x = torch.from_numpy(synth.activations(770, 1, k)).to(dev)
    outs = rq.linear_multi([w for w, _ in made], x)
    for (w, wf), y in zip(made, outs):
        assert norm_err(y.cpu().numpy(), oracle.linear_f64(x.cpu().numpy(), wf)) <= TOL_F32


@pytest.mark.parametrize("m", [2, 3])
def test_two_and_three_f32_rows_on_long_rows(dev, m):
    # Q4_K 4096 x 14336 (k > 8192 on n >= 4096): no VALU layout takes two or
    # three rows, so the f32 matrix-core kernel does (no dequantized copy)
    n, k = 4096, 14336
    w, wf = make(rq.Q4_K, n, k, 800 + m)
    x = torch.from_numpy(synth.activations(801, m, k))
    y = w.forward(x.to(dev)).cpu().numpy()
    assert norm_err(y, oracle.linear_f64(x.numpy(), wf)) <= TOL_F32


def test_gemv_walks_several_row_groups(dev):
    # An M = 1 LM head of 151936 rows: more row groups than workgroups, so
    # each workgroup walks several with the next group's loads in flight
    n, k = 151936, 896
    b = bias_vec(n, 812, torch.float32, dev)
    for qt in (rq.Q8_0, rq.Q4_K):
        w, wf = make(qt, n, k, 810 + qt)
        x = synth.activations(811, 1, k)
        r = oracle.linear_f64(x, wf)
        y = w.forward(torch.from_numpy(x).to(dev)).cpu().numpy()
        assert norm_err(y, r) <= TOL_F32, qt
        yb = w.forward(torch.from_numpy(x).to(dev), bias=b).cpu().numpy()
        assert norm_err(yb, r + b.double().cpu().numpy()[None, :]) <= TOL_F32, qt
        w.close()


@pytest.mark.parametrize("qtype,n,k", [(rq.Q4_K, 8, 160), (rq.Q8_0, 2, 48), (rq.Q6_K, 4, 192),
                                       (rq.Q5_0, 96, 32), (rq.Q4_0, 3, 96)])
@pytest.mark.parametrize("m", [1, 2, 7])
def test_generic_kernel_odd_shapes(dev, qtype, n, k, m):
    # rows cut inside a 64-element chunk: the generic kernel, exact weights,
    # f32 accumulation, f16 activations too
    w, wf = make(qtype, n, k, 820 + k + m)
    for xdt in (torch.float32, torch.float16):
        x = torch.from_numpy(synth.activations(821 + m, m, k)).to(xdt)
        y = w.forward(x.to(dev), out_dtype=torch.float32).cpu().numpy()
        assert norm_err(y, oracle.linear_f64(x.float().numpy(), wf)) <= TOL_F32


def _replay_check(fn, ref, replays=4):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm up on the capture stream (its workspace grows here)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            out = fn()
    torch.cuda.synchronize()
    for i in range(replays):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"
        # eager work between replays, on the default stream
        ref2 = fn()
        torch.cuda.synchronize()
        assert torch.equal(ref2, ref)
    return g


def test_split_k_workspace_under_graph_capture(dev):
    # The down projection at M = 512 splits K four ways into f32 partials in
    # the stream's workspace; captured, the graph refers to that workspace.
    n, k, m = 2048, 8192, 512
    w, _ = make(rq.Q6_K, n, k, 830)
    x = torch.from_numpy(synth.activations(831, m, k)).to(torch.bfloat16).to(dev)
    b = bias_vec(n, 832, torch.bfloat16, dev)
    ref = w.forward(x, bias=b)
    torch.cuda.synchronize()
    _replay_check(lambda: w.forward(x, bias=b), ref)


@pytest.mark.parametrize("m", [16, 64])
def test_small_m_split_k_under_graph_capture(dev, m):
    # The 896 x 4864 down projection at small M splits K over eight
    # workgroups per row tile; the last to finish adds the partials (in a
    # fixed order) and leaves its counter at zero for the next call or
    # replay.  Results equal the eager ones on every replay.
    n, k = 896, 4864
    w, wf = make(rq.Q4_K, n, k, 860 + m)
    x = torch.from_numpy(synth.activations(861, m, k)).to(torch.bfloat16).to(dev)
    ref = w.forward(x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert norm_err(ref.cpu().numpy(), oracle.linear_f64(x.float().cpu().numpy(), wf)) <= TOL_BF16
    for _ in range(3):  # deterministic: the same bits on every call
        assert torch.equal(w.forward(x, out_dtype=torch.float32), ref)
    _replay_check(lambda: w.forward(x, out_dtype=torch.float32), ref)


@pytest.mark.parametrize("m,n,k", [(4, 896, 4864), (16, 896, 4864), (64, 896, 896), (64, 4864, 896)])
def test_f32_small_m_split_k_under_graph_capture(dev, m, n, k):
    # f32 activations on the small-M kernel's two-limb variant: long rows and
    # short rows on few tiles split K over workgroups; the last workgroup of
    # a tile adds the partials in a fixed order, so eager calls and every
    # graph replay give the same bits, within 1e-3 of the oracle
    print(f"f32 split m={m} n={n} k={k}", flush=True)
    w, wf = make(rq.Q4_K, n, k, 870 + m + n)
    x = torch.from_numpy(synth.activations(871 + m, m, k)).to(dev)
    ref = w.forward(x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert norm_err(ref.cpu().numpy(), oracle.linear_f64(x.cpu().numpy(), wf)) <= TOL_F32
    for _ in range(3):
        assert torch.equal(w.forward(x, out_dtype=torch.float32), ref)
    _replay_check(lambda: w.forward(x, out_dtype=torch.float32), ref)


def test_capture_without_warmup(dev):
    # A fresh stream has no workspace yet: under capture the split-K
    # partials and the aligned copy of x come from a buffer allocated outside
    # the graph (the thread's capture mode relaxed for the allocation), which
    # the graph then refers to.
    n, k, m = 2048, 8192, 300
    w, _ = make(rq.Q4_K, n, k, 840)
    x = torch.from_numpy(synth.activations(841, m, k)).to(torch.bfloat16).to(dev)
    xv = _offset_view(x, 1)
    ref = w.forward(x)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            out = w.forward(xv)
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)


def test_embedding_refuses_capture(dev):
    w, _ = make(rq.Q8_0, 16, 64, 850)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with pytest.raises(rq.RqError) as e:
            with torch.cuda.graph(g, stream=s):
                w.embedding([1, 2])
    assert "cannot be captured" in e.value.message
    assert torch.equal(w.embedding([1, 2]).cpu(), w.dequantize()[1:3].cpu())
