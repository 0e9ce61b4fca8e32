"""The Q4_K_M prefill workload at its real shapes: M = 512 bf16 activations
through every linear of a hidden-2048 / FFN-8192 layer and the Q6_K
262144 x 2048 output projection (generate.rs:45 issues them as 512-token
prefill chunks).  Each shape runs the tile route rq_linear picks for it:

  q/k/o  Q4_K 2048 x 2048   64 x 64 tiles of two waves (32 K-steps)
  v      Q6_K 2048 x 2048   the same route with the Q6_K decoder
  gate/up Q4_K 8192 x 2048  128 x 128 tiles, unsplit, stored straight to y
  down   Q6_K 2048 x 8192   128 x 128 tiles, K split four ways (f32 partials)
  head   Q6_K 262144 x 2048 the pipelined 256 x 256 kernel, 64 K-steps,
                            XCD-aware tile order

Reference: runtimed-gguf dequant + dense matmul (linear_layer.rs:88-104),
evaluated by the oracle in f64 on the bit-exact dequantized rows of the
sampled output columns.  Column samples cover every output tile of the
route.  Gate: normalized error <= 2e-2 (bf16 operands).

The same shapes also run with f32 activations and f32 outputs, the
reference's compute type (store.rs:3-4: "Compute always runs in F32"), which
rq_linear takes on its f32 route; gate 1e-3 (f32 accumulation)."""
import numpy as np
import pytest
import torch

import oracle
from runtimed_amd import rq, synth
from tests.conftest import norm_err

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
TOL_F32 = 1e-3
M = 512

SHAPES = [
    ("q/k/o", rq.Q4_K, 2048, 2048),
    ("v", rq.Q6_K, 2048, 2048),
    ("gate/up", rq.Q4_K, 8192, 2048),
    ("down", rq.Q6_K, 2048, 8192),
    ("head", rq.Q6_K, 262144, 2048),
]


def sample_columns(n: int, tile: int, per_tile: int, seed: int) -> np.ndarray:
    """per_tile distinct columns from every tile of `tile` output columns
    (always the tile's first and last column)."""
    rng = np.random.default_rng(seed)
    cols = []
    for t0 in range(0, n, tile):
        width = min(tile, n - t0)
        pick = {0, width - 1}
        while len(pick) < min(per_tile, width):
            pick.add(int(rng.integers(width)))
        cols.extend(t0 + c for c in sorted(pick))
    return np.array(cols, dtype=np.int64)


def rows_f32(qtype: int, data: np.ndarray, k: int, rows: np.ndarray) -> np.ndarray:
    """The dequantized weight rows `rows` (k a multiple of the block size, so
    every row is a whole number of blocks), through the oracle."""
    elems, bbytes = rq.GEOMETRY[qtype]
    per_row = k // elems * bbytes
    blob = np.concatenate([data[r * per_row:(r + 1) * per_row] for r in rows])
    rc, wf = oracle.dequant_tensor(qtype, blob, len(rows) * k, threads=8)
    assert rc == 0
    return wf.reshape(len(rows), k)


@pytest.mark.parametrize("name,qtype,n,k", SHAPES, ids=[s[0] for s in SHAPES])
def test_prefill_m512_real_shape(dev, name, qtype, n, k):
    print(f"prefill m={M} {name} qtype={qtype} n={n} k={k}", flush=True)
    data = synth.weight_blocks(qtype, 900 + n + k, n, k)
    w = rq.QWeight(qtype, data, n, k)
    x32 = torch.from_numpy(synth.activations(910 + n, M, k))
    xb = x32.to(torch.bfloat16)
    if n <= 2048:
        cols = np.arange(n)
    elif n <= 8192:
        cols = sample_columns(n, 128, 16, n)
    else:
        cols = sample_columns(n, 256, 2, n)
    wrows = rows_f32(qtype, data, k, cols)
    r = oracle.linear_f64(xb.float().numpy(), wrows)
    xd = xb.to(dev)
    for ydt in (torch.bfloat16, torch.float32):
        y = w.forward(xd, out_dtype=ydt)
        torch.cuda.synchronize()
        ys = y[:, torch.from_numpy(cols).to(dev)].float().cpu().numpy()
        err = norm_err(ys, r)
        print(f"  {name} y={ydt} normalized error {err:.2e} on {len(cols)} columns", flush=True)
        assert err <= TOL_BF16, (name, ydt, err)
        del y
    del xd
    r32 = oracle.linear_f64(x32.numpy(), wrows)
    y = w.forward(x32.to(dev), out_dtype=torch.float32)
    torch.cuda.synchronize()
    err = norm_err(y[:, torch.from_numpy(cols).to(dev)].cpu().numpy(), r32)
    print(f"  {name} x=f32 y=f32 normalized error {err:.2e} on {len(cols)} columns", flush=True)
    assert err <= TOL_F32, (name, "f32", err)
    del y
    w.close()
