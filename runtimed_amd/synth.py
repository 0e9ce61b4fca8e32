"""Seeded synthetic GGUF tensors and activations for tests and benchmarks.

One portable generator: splitmix64 as in runtimed's sampler Rng
(crates/runtimed-core/src/engine/generator.rs:51-61), evaluated in closed form
for every stream position (z_i = mix(seed + (i + 1) * golden)), plus
Box-Muller for normal variates.  The same seed gives the same bytes on every
machine.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def u64(seed: int, n: int, stream: int = 0) -> np.ndarray:
    """n splitmix64 outputs of the stream (seed, stream)."""
    base = np.uint64((seed * 0x100000001B3 + stream * 0xD1342543DE82EF95) & 0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        z = base + (np.arange(1, n + 1, dtype=np.uint64) * _GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform(seed: int, n: int, lo: float = 0.0, hi: float = 1.0, stream: int = 0) -> np.ndarray:
    """float64 uniforms in [lo, hi)."""
    u = (u64(seed, n, stream) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    return lo + (hi - lo) * u


def normal(seed: int, n: int, stream: int = 0) -> np.ndarray:
    """float64 N(0, 1) variates by Box-Muller."""
    h = (n + 1) // 2
    u1 = 1.0 - uniform(seed, h, stream=stream * 2 + 1)  # (0, 1]
    u2 = uniform(seed, h, stream=stream * 2 + 2)
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * h)
    out[0::2] = r * np.cos(2.0 * np.pi * u2)
    out[1::2] = r * np.sin(2.0 * np.pi * u2)
    return out[:n]


def random_bytes(seed: int, n: int, stream: int = 0) -> np.ndarray:
    return u64(seed, (n + 7) // 8, stream).view(np.uint8)[:n].copy()


def f16_bits(v: np.ndarray) -> np.ndarray:
    return np.asarray(v, dtype=np.float32).astype(np.float16).view(np.uint16)


def q8_0_blocks(seed: int, nblocks: int) -> np.ndarray:
    """Q8_0: d = f16(U(0.001, 0.02)), 32 int8 quants ~ U[-127, 127]."""
    out = np.empty((nblocks, 34), dtype=np.uint8)
    out[:, 0:2] = f16_bits(uniform(seed, nblocks, 0.001, 0.02, stream=1)).view(np.uint8).reshape(-1, 2)
    q = (u64(seed, nblocks * 32, stream=2) % np.uint64(255)).astype(np.int16) - 127
    out[:, 2:] = q.astype(np.int8).view(np.uint8).reshape(nblocks, 32)
    return out.reshape(-1)


def q4_k_blocks(seed: int, nblocks: int) -> np.ndarray:
    """Q4_K: d, dmin = f16(U(1e-4, 1e-2)); 12 scale bytes and 128 qs bytes uniform."""
    out = random_bytes(seed, nblocks * 144, stream=3).reshape(nblocks, 144)
    out[:, 0:2] = f16_bits(uniform(seed, nblocks, 1e-4, 1e-2, stream=4)).view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = f16_bits(uniform(seed, nblocks, 1e-4, 1e-2, stream=5)).view(np.uint8).reshape(-1, 2)
    return out.reshape(-1)


def q6_k_blocks(seed: int, nblocks: int) -> np.ndarray:
    """Q6_K: ql, qh, int8 scales uniform bytes; d = f16(U(1e-4, 1e-2)) (finite)."""
    out = random_bytes(seed, nblocks * 210, stream=6).reshape(nblocks, 210)
    out[:, 208:210] = f16_bits(uniform(seed, nblocks, 1e-4, 1e-2, stream=7)).view(np.uint8).reshape(-1, 2)
    return out.reshape(-1)


def q5_k_blocks(seed: int, nblocks: int) -> np.ndarray:
    out = random_bytes(seed, nblocks * 176, stream=8).reshape(nblocks, 176)
    out[:, 0:2] = f16_bits(uniform(seed, nblocks, 1e-4, 1e-2, stream=9)).view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = f16_bits(uniform(seed, nblocks, 1e-4, 1e-2, stream=10)).view(np.uint8).reshape(-1, 2)
    return out.reshape(-1)


def q4_0_blocks(seed: int, nblocks: int) -> np.ndarray:
    out = random_bytes(seed, nblocks * 18, stream=11).reshape(nblocks, 18)
    out[:, 0:2] = f16_bits(uniform(seed, nblocks, 1e-3, 2e-2, stream=12)).view(np.uint8).reshape(-1, 2)
    return out.reshape(-1)


def q5_0_blocks(seed: int, nblocks: int) -> np.ndarray:
    out = random_bytes(seed, nblocks * 22, stream=13).reshape(nblocks, 22)
    out[:, 0:2] = f16_bits(uniform(seed, nblocks, 1e-3, 2e-2, stream=14)).view(np.uint8).reshape(-1, 2)
    return out.reshape(-1)


BLOCKS = {8: q8_0_blocks, 12: q4_k_blocks, 14: q6_k_blocks, 13: q5_k_blocks, 2: q4_0_blocks,
          6: q5_0_blocks}
GEOMETRY = {2: (32, 18), 6: (32, 22), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


def weight_blocks(qtype: int, seed: int, n: int, k: int) -> np.ndarray:
    elems, _ = GEOMETRY[qtype]
    assert (n * k) % elems == 0
    return BLOCKS[qtype](seed, n * k // elems)


def activations(seed: int, m: int, k: int) -> np.ndarray:
    """float32 N(0, 1) activations [m, k]."""
    return normal(seed, m * k, stream=20).astype(np.float32).reshape(m, k)


def fp8_weight_values(seed: int, n: int, k: int) -> np.ndarray:
    """float32 N(0, 1) clipped to +-448, to be encoded as e4m3 weight codes."""
    return np.clip(normal(seed, n * k, stream=21), -448.0, 448.0).astype(np.float32).reshape(n, k)


def fp8_row_scales(seed: int, n: int) -> np.ndarray:
    """Per-output-row scales ~ U(0.5, 2) / 448."""
    return (uniform(seed, n, 0.5, 2.0, stream=22) / 448.0).astype(np.float32)
