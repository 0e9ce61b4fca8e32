"""Pins the oracle's Marlin INT4 and paged-KV quantizer functions.

Checks:
  * the reference's own tests, transcribed: marlin_gemv.rs:209-222 (repack,
    resident bytes, y = x deq^T), linear_layer.rs:143-160 ([10, 14]),
    quantize.rs:142-200 (FP8 / INT8 round trips within 0.2, scale shapes);
  * closed forms of the formats: the packed word of a hand-quantized row,
    Rust's round-half-away-from-zero at exact ties, clamps at 0 / 15 and
    -128 / 127, NaN -> 0, the 1e-12 and 1e-8 floors, per-head maxima over
    every batch, NaN skipped by the maximum;
  * an independent numpy restatement (tests/reference_np.py style) of the
    nibble layout and of the per-head scales on seeded random tensors.
"""
import numpy as np
import pytest

import oracle


def np_marlin_repack(w, s):
    """Independent restatement of marlin_gemv.rs:66-97 in numpy."""
    n, k = w.shape
    kc = (k + 31) // 32
    inv = np.where(np.abs(s) > np.float32(1e-12), np.float32(1) / s, np.float32(1)).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        t = w.astype(np.float32) * inv[:, None]
        # half away from zero; |t| + 0.5 is exact in double for every f32 |t|
        r = np.sign(t) * np.floor(np.abs(t).astype(np.float64) + 0.5)
        q = r.astype(np.float32) + np.float32(8)
        q = np.where(np.isnan(q), 0, np.clip(q, 0, 15)).astype(np.uint32)
    qp = np.full((n, kc * 32), 8, dtype=np.uint32)
    qp[:, :k] = q
    qp = qp.reshape(n, kc, 4, 8)
    words = np.zeros((n, kc, 4), dtype=np.uint32)
    for i in range(8):
        words |= qp[..., i] << np.uint32(4 * i)
    return words.transpose(1, 0, 2).copy()


def test_marlin_reference_kat():  # marlin_gemv.rs:209-222
    w = np.array([[1.0, -2.0, 3.0, 0.0], [0.5, 1.5, -0.5, 2.0]], np.float32)
    s = np.array([0.5, 0.25], np.float32)
    p = oracle.marlin_repack(w, s)
    assert p.shape == (1, 2, 4)
    assert p.nbytes + s.nbytes == (2 * 4) * 4 + 2 * 4  # resident_bytes
    # hand-quantized: row 0 = w/0.5 + 8 = [10, 4, 14, 8]; row 1 = w/0.25 + 8
    # = [10, 14, 6, 16 -> 15]; the 28 padding inputs hold 8
    assert p[0, 0].tolist() == [0x88888E4A, 0x88888888, 0x88888888, 0x88888888]
    assert p[0, 1].tolist() == [0x8888F6EA, 0x88888888, 0x88888888, 0x88888888]
    d = oracle.marlin_dequant(p, s, 4)
    assert d.tolist() == [[1.0, -2.0, 3.0, 0.0], [0.5, 1.5, -0.5, 1.75]]
    y = oracle.marlin_gemv_f64(np.array([[2.0, 1.0, -1.0, 3.0]], np.float32), p, s)
    assert y.tolist() == [[-3.0, 8.25]]


def test_linear_marlin_kat():  # linear_layer.rs:143-160
    w = np.array([[1.0, 2.0, 3.0, 4.0], [2.0, 3.0, 4.0, 5.0]], np.float32)
    p = oracle.marlin_repack(w, np.ones(2, np.float32))
    y = oracle.marlin_gemv_f64(np.ones((1, 4), np.float32), p, np.ones(2, np.float32))
    assert y.tolist() == [[10.0, 14.0]]


def test_marlin_rounding_clamps_and_floors():
    # s = 0.5: w / s = [0.5, -0.5, 1.5, 2.5, -2.5, 100, -100, nan, inf, -inf]
    w = np.array([[0.25, -0.25, 0.75, 1.25, -1.25, 50, -50, np.nan, np.inf, -np.inf]], np.float32)
    p = oracle.marlin_repack(w, np.array([0.5], np.float32))
    d = oracle.marlin_dequant(p, np.ones(1, np.float32), 10)
    # half away from zero (a half-even rounding gives 0, 0, 2, 2, -2)
    assert d[0].tolist() == [1, -1, 2, 3, -3, 7, -8, -8, 7, -8]
    # |s| <= 1e-12 divides by 1, and so does a NaN scale
    for s in (0.0, 1e-13, -1e-13, np.nan):
        p = oracle.marlin_repack(np.array([[3.0, -2.6]], np.float32), np.array([s], np.float32))
        d = oracle.marlin_dequant(p, np.ones(1, np.float32), 2)
        assert d[0].tolist() == [3.0, -3.0]


def test_marlin_matches_numpy_restatement():
    rng = np.random.default_rng(7)
    for n, k in [(5, 50), (32, 64), (17, 100), (64, 896)]:
        w = rng.standard_normal((n, k)).astype(np.float32) * 3
        s = (rng.uniform(0.05, 0.6, n) * rng.choice([-1, 1], n)).astype(np.float32)
        p = oracle.marlin_repack(w, s)
        assert np.array_equal(p, np_marlin_repack(w, s))
        # dequant layout: nibble k % 8 of word (k % 32) / 8 of record [k / 32][row]
        words = rng.integers(0, 2**32, p.shape, dtype=np.uint64).astype(np.uint32)
        d = oracle.marlin_dequant(words, s, k)
        kk = np.arange(k)
        nib = (words[kk // 32, :, (kk % 32) // 8] >> (4 * (kk % 8)).astype(np.uint32)[:, None]) & 15
        want = (nib.T.astype(np.int32) - 8).astype(np.float32) * s[:, None]
        assert np.array_equal(d, want)
        x = rng.standard_normal((3, k)).astype(np.float32)
        y = oracle.marlin_gemv_f64(x, words, s)
        ref = (x.astype(np.float64) @ ((nib.T.astype(np.float64) - 8)).T) * s.astype(np.float64)
        assert np.allclose(y, ref, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------- KV cache -----

def test_kv_roundtrips():  # quantize.rs:142-200
    data = ((np.arange(64) - 32) * 0.1).astype(np.float32).reshape(1, 2, 2, 16)
    for int8 in (False, True):
        q, s = oracle.kv_quantize(data, int8)
        assert q.shape == data.shape and s.shape == (2,)
        rec = oracle.kv_dequantize(q, s, int8)
        assert np.all(np.abs(rec - data) < 0.2)
    data = (np.arange(64) * 0.05).astype(np.float32).reshape(1, 2, 2, 16)
    q, s = oracle.kv_quantize(data)
    assert np.all(np.abs(oracle.kv_dequantize(q, s) - data) < 0.2)


def test_kv_scales_closed_form():
    rng = np.random.default_rng(3)
    t = rng.standard_normal((3, 4, 5, 8)).astype(np.float32)
    t[2, 1, 0, 0] = 9.0          # head 1's maximum sits in the last batch
    t[0, 3, 4, 7] = np.nan       # skipped by the maximum
    for int8, d in ((False, 448.0), (True, 127.0)):
        _, s = oracle.kv_quantize(t, int8)
        a = np.abs(np.nan_to_num(t, nan=0.0))
        want = np.maximum(a.max(axis=(0, 2, 3)) / np.float32(d), np.float32(1e-8)).astype(np.float32)
        assert np.array_equal(s, want)
        assert s[1] == np.float32(9.0) / np.float32(d)
    _, s = oracle.kv_quantize(np.zeros((1, 2, 3, 4), np.float32))
    assert s.tolist() == [np.float32(1e-8)] * 2


def test_kv_codes_closed_form():
    # max|t| = 448 (FP8) or 127 (INT8) makes the scale exactly 1
    v = np.array([448.0, 1.0, 1.0625, -2.5, 0.5, -0.5, 2.5, -448.0, np.nan], np.float32)
    q, s = oracle.kv_quantize(v.reshape(1, 1, 1, -1))
    assert s.tolist() == [1.0]
    # 1.0625 lies halfway between 1.0 (0x38) and 1.125 (0x39): ties go low
    assert q.ravel().tolist()[:8] == [0x7E, 0x38, 0x38, 0xC2, 0x30, 0xB0, 0x42, 0xFE]
    assert q.ravel()[8] == 0x7F
    v = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 126.5, np.nan], np.float32)
    q, s = oracle.kv_quantize(v.reshape(1, 1, 1, -1), int8=True)
    assert s.tolist() == [1.0]
    # round half away from zero; NaN -> 0
    assert q.view(np.int8).ravel().tolist() == [127, 3, -3, 1, -1, 127, 0]
    rec = oracle.kv_dequantize(q, s, int8=True)
    assert rec.ravel().tolist() == [127.0, 3.0, -3.0, 1.0, -1.0, 127.0, 0.0]


def test_kv_non_4d_is_one_head():  # quantize.rs:14-18
    t = np.linspace(-3, 5, 40, dtype=np.float32).reshape(5, 8)
    q, s = oracle.kv_quantize(t)
    assert s.shape == (1,) and s[0] == np.float32(5.0) / np.float32(448.0)
    assert q.shape == (5, 8)
