"""Quantized embedding rows (rq_embedding) -- the quantized branch of
Weights::embed / Weights::candidate_weights (embed_layer.rs:16-84): each
requested row is the bit-exact dequant of that row of the flat GGUF stream,
i.e. the oracle's dequant_tensor (dequant.rs:83-146) indexed by id."""
import numpy as np
import pytest
import torch

import oracle
from runtimed_amd import rq, synth

pytestmark = pytest.mark.gpu

ALL = [rq.Q8_0, rq.Q4_0, rq.Q5_0, rq.Q4_K, rq.Q5_K, rq.Q6_K]


def bits_equal(got: np.ndarray, want: np.ndarray):
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("qtype", ALL)
@pytest.mark.parametrize("n,k", [(512, 896), (96, 2048), (3, 256)])
def test_rows_bit_exact(dev, qtype, n, k):
    blocks = synth.weight_blocks(qtype, 61 + n, n, k)
    rc, wf = oracle.dequant_tensor(qtype, blocks, n * k)
    assert rc == 0
    w = rq.QWeight(qtype, blocks, n, k)
    rng = np.random.default_rng(n + k)
    ids = np.concatenate([[0, n - 1, n - 1], rng.integers(0, n, 29)]).astype(np.uint32)
    got = w.embedding(ids).cpu().numpy()
    assert got.shape == (ids.size, k)
    bits_equal(got, wf.reshape(n, k)[ids])


@pytest.mark.parametrize("qtype", ALL)
def test_random_bytes_rows(dev, qtype):
    # raw random block bytes: f16 scales may be Inf or NaN, kept as the
    # reference keeps them
    elems, bsz = oracle.geometry(qtype)
    n, k = 64, 512
    data = synth.random_bytes(71, n * k // elems * bsz)
    rc, wf = oracle.dequant_tensor(qtype, data, n * k)
    assert rc == 0
    w = rq.QWeight(qtype, data, n, k)
    ids = np.arange(n, dtype=np.uint32)[::-3]
    bits_equal(w.embedding(ids).cpu().numpy(), wf.reshape(n, k)[ids])


def test_embed_kat(dev):
    # embed_layer.rs:92-125 looks up ids [1, 3] of the table row r = [3r, 3r+1,
    # 3r+2]; here the same rows, 32 wide, as Q8_0 blocks with d = 1 and q = 3r + i.
    blocks = bytearray()
    for r in range(4):
        blocks += np.array([0x3C00], dtype="<u2").tobytes()
        blocks += np.array([3 * r + i for i in range(32)], dtype=np.int8).tobytes()
    w = rq.QWeight(rq.Q8_0, np.frombuffer(bytes(blocks), dtype=np.uint8), 4, 32)
    got = w.embedding([1, 3]).cpu().numpy()
    assert got.shape == (2, 32)
    assert got[0, :3].tolist() == [3.0, 4.0, 5.0]
    assert got[1, :3].tolist() == [9.0, 10.0, 11.0]


def test_empty_and_out_of_range(dev):
    n, k = 8, 256
    w = rq.QWeight(rq.Q4_K, synth.weight_blocks(rq.Q4_K, 3, n, k), n, k)
    assert tuple(w.embedding([]).shape) == (0, k)
    with pytest.raises(rq.RqError) as e:
        w.embedding([2, n])
    assert e.value.code == -5 and "out of range" in str(e.value)
