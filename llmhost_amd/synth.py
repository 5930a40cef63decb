"""Seeded synthetic operands for the block-quantized matmul workloads.

Counter-based SplitMix64 (Steele, Lea, Flood 2014), vectorised in numpy, so
any slice of a stream can be regenerated independently.  Distributions:
  * Q4 codes: raw 4-bit patterns uniform in 0..15 (two's-complement -8..7);
  * Q8_0 codes: uniform integers in [-127, 127];
  * block scales: uniform f32 in [1e-3, 2e-2], rounded to f16 (RNE);
  * activations: f32 N(0, 1) by Box-Muller on two 53-bit uniforms;
  * ragged batches: sequence lengths uniform in 1..8, packed to M rows.
"""

from __future__ import annotations

import numpy as np

from .formats import BLOCK_Q4, BLOCK_Q8_0

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, count: int, offset: int = 0) -> np.ndarray:
    """Outputs offset..offset+count-1 of the SplitMix64 stream for `seed`."""
    with np.errstate(over="ignore"):
        idx = np.arange(offset + 1, offset + count + 1, dtype=np.uint64)
        z = np.uint64(seed) + idx * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform01(seed: int, count: int, offset: int = 0) -> np.ndarray:
    """float64 uniforms in [0, 1) from the top 53 bits."""
    return (splitmix64(seed, count, offset) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def normal_f32(seed: int, count: int) -> np.ndarray:
    """f32 N(0, 1) via Box-Muller (u1 in (0, 1], u2 in [0, 1))."""
    half = (count + 1) // 2
    u1 = 1.0 - uniform01(seed, half, 0)
    u2 = uniform01(seed, half, half)
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * half, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return z[:count].astype(np.float32)


def scales_f16(seed: int, count: int, lo: float = 1e-3, hi: float = 2e-2) -> np.ndarray:
    """f16 bit patterns of uniform [lo, hi] scales."""
    s = (lo + uniform01(seed, count) * (hi - lo)).astype(np.float32)
    return s.astype(np.float16).view(np.uint16)


def q4_blocks(seed: int, n: int, k: int) -> np.ndarray:
    """Row-major BlockQ4[n][k/32] with uniform nibbles and f16 scales."""
    assert k % 32 == 0
    nb = n * (k // 32)
    out = np.empty(nb, dtype=BLOCK_Q4)
    raw = splitmix64(seed, 2 * nb).view(np.uint8).reshape(nb, 16)
    out["qs"] = raw
    out["scale"] = scales_f16(seed ^ 0x5CA1E, nb)
    return out


def q8_blocks(seed: int, n: int, k: int) -> np.ndarray:
    """Row-major BlockQ8_0[n][k/32], codes uniform in [-127, 127]."""
    assert k % 32 == 0
    nb = n * (k // 32)
    out = np.empty(nb, dtype=BLOCK_Q8_0)
    z = splitmix64(seed, nb * 32) >> np.uint64(32)
    out["qs"] = ((z * np.uint64(255)) >> np.uint64(32)).astype(np.int64).reshape(nb, 32) - 127
    out["scale"] = scales_f16(seed ^ 0x5CA1E, nb)
    return out


def activations(seed: int, m: int, k: int) -> np.ndarray:
    """f32 N(0, 1) activations [m, k]."""
    return normal_f32(seed, m * k).reshape(m, k)


def ragged_lengths(seed: int, m: int, lo: int = 1, hi: int = 8) -> list[int]:
    """Sequence lengths uniform in lo..hi packed until they sum to m rows
    (the last sequence is truncated)."""
    out, total, i = [], 0, 0
    while total < m:
        u = uniform01(seed, 1, i)[0]
        ln = lo + int(u * (hi - lo + 1))
        ln = min(ln, m - total)
        out.append(ln)
        total += ln
        i += 1
    return out
