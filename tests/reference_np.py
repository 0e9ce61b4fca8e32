"""Independent numpy restatements of the GGML block formats.

Written from the published GGML block layouts (ggml-common.h / ggml-quants.c
as described in GGUF's format documentation), vectorised over blocks and
structured differently from the scalar loops of the C oracle, so that a
dropped term, a wrong shift or a transposed index in either one shows up as
a bit mismatch.  Test infrastructure only.
"""
from __future__ import annotations

import numpy as np


def f16(b: np.ndarray) -> np.ndarray:
    """Little-endian f16 byte pairs [..., 2] -> float32 (numpy's IEEE widening)."""
    return np.ascontiguousarray(b).view(np.float16)[..., 0].astype(np.float32)


def q8_0(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 34)
    d = f16(b[:, 0:2])
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (d[:, None] * q).reshape(-1)


def q4_0(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 18)
    d = f16(b[:, 0:2])
    qs = b[:, 2:]
    q = np.concatenate([qs & 0x0F, qs >> 4], axis=1).astype(np.float32) - 8.0
    return (d[:, None] * q).reshape(-1)


def q5_0(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 22)
    d = f16(b[:, 0:2])
    qh = b[:, 2:6].copy().view("<u4")[:, 0]
    bits = ((qh[:, None] >> np.arange(32, dtype=np.uint32)) & 1).astype(np.uint8)
    qs = b[:, 6:]
    lo = np.concatenate([qs & 0x0F, qs >> 4], axis=1)
    q = (lo | (bits << 4)).astype(np.float32) - 16.0
    return (d[:, None] * q).reshape(-1)


def _k4_scales(sc: np.ndarray):
    """The 8 (scale, min) 6-bit pairs of a K-quant super-block, [nb, 8] each."""
    s = sc.astype(np.uint16)
    scale = np.empty((s.shape[0], 8), dtype=np.uint16)
    mins = np.empty_like(scale)
    scale[:, :4] = s[:, 0:4] & 63
    mins[:, :4] = s[:, 4:8] & 63
    scale[:, 4:] = (s[:, 8:12] & 0x0F) | ((s[:, 0:4] >> 6) << 4)
    mins[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return scale.astype(np.float32), mins.astype(np.float32)


def q4_k(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 144)
    nb = b.shape[0]
    d, dmin = f16(b[:, 0:2]), f16(b[:, 2:4])
    scale, mins = _k4_scales(b[:, 4:16])
    qs = b[:, 16:].reshape(nb, 4, 32)
    # sub-block 2c = low nibbles of chunk c, 2c+1 = high nibbles
    q = np.stack([qs & 0x0F, qs >> 4], axis=2).reshape(nb, 8, 32).astype(np.float32)
    a = d[:, None] * scale
    m = dmin[:, None] * mins
    return (a[:, :, None] * q - m[:, :, None]).astype(np.float32).reshape(-1)


def q5_k(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 176)
    nb = b.shape[0]
    d, dmin = f16(b[:, 0:2]), f16(b[:, 2:4])
    scale, mins = _k4_scales(b[:, 4:16])
    qh = b[:, 16:48]
    qs = b[:, 48:].reshape(nb, 4, 32)
    lo = np.stack([qs & 0x0F, qs >> 4], axis=2).reshape(nb, 8, 32)
    hb = np.stack([(qh >> s) & 1 for s in range(8)], axis=1)  # sub-block s uses qh bit s
    q = lo.astype(np.float32) + 16.0 * hb.astype(np.float32)
    a = d[:, None] * scale
    m = dmin[:, None] * mins
    return (a[:, :, None] * q - m[:, :, None]).astype(np.float32).reshape(-1)


def q6_k(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 210)
    nb = b.shape[0]
    ql = b[:, 0:128].reshape(nb, 2, 64)
    qh = b[:, 128:192].reshape(nb, 2, 32)
    sc = b[:, 192:208].view(np.int8).reshape(nb, 2, 8).astype(np.float32)
    d = f16(b[:, 208:210])
    lo = np.concatenate([ql[:, :, :32] & 0x0F, ql[:, :, 32:] & 0x0F, ql[:, :, :32] >> 4,
                         ql[:, :, 32:] >> 4], axis=2)  # [nb, 2, 128] in output order
    hi = np.concatenate([(qh >> (2 * j)) & 3 for j in range(4)], axis=2)
    q = (lo | (hi << 4)).astype(np.float32) - 32.0
    # output index l + 32 j of a half uses scale 2 j + l // 16
    l = np.arange(128)
    sidx = 2 * (l // 32) + (l % 32) // 16
    scale = sc[:, :, sidx]
    ds = d[:, None, None] * scale
    return (ds * q).astype(np.float32).reshape(-1)


DECODERS = {8: q8_0, 2: q4_0, 6: q5_0, 12: q4_k, 13: q5_k, 14: q6_k}


def e4m3_table() -> np.ndarray:
    """All 256 OCP e4m3fn values computed from the format definition."""
    b = np.arange(256)
    sign = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = (b & 7).astype(np.float64)
    v = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    v = sign * v
    v[(e == 15) & ((b & 7) == 7)] = np.nan
    return v.astype(np.float32)


def e4m3_nearest_tie_low(x: np.ndarray) -> np.ndarray:
    """Brute force: nearest non-negative code by |value - |x||, ties to the
    smaller code, |x| >= 448 -> 0x7e, NaN -> 0x7f, sign bit copied."""
    x = np.asarray(x, dtype=np.float32)
    pos = e4m3_table()[:127].astype(np.float64)
    a = np.abs(x).astype(np.float64)
    dist = np.abs(pos[None, :] - a[:, None])
    code = np.argmin(dist, axis=1).astype(np.uint8)  # argmin keeps the first (lower) on ties
    code = np.where(a >= 448.0, 0x7E, code).astype(np.uint8)
    code = np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)
    return np.where(np.isnan(x), 0x7F, code).astype(np.uint8)
