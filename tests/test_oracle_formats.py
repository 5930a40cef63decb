"""Pins of the oracle's llm-quant restatement (crates/llm-quant/src/lib.rs).

The reference's own tests (lib.rs:147-222) are re-created with their formula
inputs; the rest pins each function against a library routine or a closed
form chosen so that a plausible slip (half-even instead of half-away
rounding, a missing clamp, swapped nibble halves, a wrong f16 rounding) fails.
"""

import numpy as np
import pytest

from llmhost_amd.formats import BLOCK_Q4, q4_from_nibbles, q4_nibbles


# ---- f16 <-> f32 (half 2.7.1): pinned against numpy's IEEE binary16 ---------
def test_f16_to_f32_all_patterns(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(b) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne_matches_numpy(oracle):
    rng = np.random.default_rng(7)
    vals = [rng.uniform(-70000, 70000, 3000), rng.uniform(-1, 1, 3000) * 1e-3,
            rng.uniform(-1, 1, 3000) * 1e-6, rng.uniform(1e-3, 2e-2, 3000)]
    # Exact midpoints between adjacent f16 values: ties must go to even.
    h = np.arange(0, 0x7bff, 37, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32)
    vals += [mids, -mids, np.array([0.0, -0.0, 65504, 65520, 65519.99, 1e9, 5.96e-8, 2.98e-8,
                                    2.99e-8, 1e-9, np.inf, -np.inf], dtype=np.float32)]
    x = np.concatenate([np.asarray(v, dtype=np.float32) for v in vals])
    ref = x.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(v) for v in x], dtype=np.uint16)
    assert np.array_equal(got, ref)


# ---- nibble decode: brute force against the textbook two's-complement value ---
def test_nibble_decode_brute_force(oracle):
    for byte in range(256):
        blk = np.zeros(1, dtype=BLOCK_Q4)
        blk["qs"][0, 3] = byte
        lo, hi = byte & 0xF, byte >> 4
        assert oracle.q4_nibble(blk, 6) == (lo - 16 if lo >= 8 else lo)
        assert oracle.q4_nibble(blk, 7) == (hi - 16 if hi >= 8 else hi)
    # formats.py's numpy decode/encode agrees with the oracle on random blocks
    rng = np.random.default_rng(3)
    blocks = np.zeros(64, dtype=BLOCK_Q4)
    blocks["qs"] = rng.integers(0, 256, (64, 16), dtype=np.uint8)
    nib = q4_nibbles(blocks)
    for b in range(0, 64, 7):
        assert [oracle.q4_nibble(blocks[b], i) for i in range(32)] == list(nib[b])
    assert np.array_equal(q4_from_nibbles(nib, blocks["scale"])["qs"], blocks["qs"])


# ---- the reference's own tests (lib.rs:147-222) --------------------------------
def _pattern():
    src = (np.arange(32, dtype=np.float32) * np.float32(0.37) - np.float32(5.1)).astype(np.float32)
    src[0], src[1], src[2] = -6.0, 6.0, 0.0
    return src


def test_q8_0_roundtrip(oracle):
    src = _pattern()
    back = oracle.dequantize_q8_0(oracle.quantize_q8_0(src))
    amax = np.abs(src).max()
    assert np.abs(src - back).max() <= amax / 127 + 1e-3


def test_q4_roundtrip(oracle):
    src = _pattern()
    blk = oracle.quantize_q4(src)
    back = oracle.dequantize_q4(blk)
    amax = np.abs(src).max()
    assert np.abs(src - back).max() <= amax / 8 + 1e-3
    assert all(-8 <= oracle.q4_nibble(blk[0], i) <= 7 for i in range(32))


def test_zero_block(oracle):
    z = np.zeros(32, dtype=np.float32)
    assert np.all(oracle.dequantize_q8_0(oracle.quantize_q8_0(z)) == 0)
    assert np.all(oracle.dequantize_q4(oracle.quantize_q4(z)) == 0)
    assert oracle.quantize_q4(z)["scale"][0] == 0 and oracle.quantize_q8_0(z)["scale"][0] == 0


def test_slice_helpers_roundtrip(oracle):
    src = (np.sin(np.arange(96, dtype=np.float32)) * 3.0).astype(np.float32)
    assert np.abs(oracle.dequantize_q8_0(oracle.quantize_q8_0(src)) - src).max() < 0.05
    assert np.abs(oracle.dequantize_q4(oracle.quantize_q4(src)) - src).max() < 0.5
    with pytest.raises(ValueError):
        oracle.quantize_q4(np.zeros(33, dtype=np.float32))


# ---- closed-form special cases ---------------------------------------------------
def test_q4_quantize_ties_round_away_and_clamp(oracle):
    # amax = 8 -> scale = f16(1.0) exactly -> inv = 1: codes are round(v).
    src = np.zeros(32, dtype=np.float32)
    src[:10] = [8.0, -8.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 6.5, -7.5]
    blk = oracle.quantize_q4(src)
    assert blk["scale"][0] == np.float16(1.0).view(np.uint16)
    got = [oracle.q4_nibble(blk[0], i) for i in range(10)]
    # +8 clamps to 7; halves go away from zero (rint would give 2, -2, 0, -0, ...)
    assert got == [7, -8, 3, -3, 1, -1, 2, -2, 7, -8]


def test_q8_quantize_ties_round_away_and_scale_rounding(oracle):
    # amax = 127 -> scale = f16(1.0) -> inv = 1.
    src = np.zeros(32, dtype=np.float32)
    src[:8] = [127.0, -127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -3.5]
    blk = oracle.quantize_q8_0(src)
    assert blk["scale"][0] == np.float16(1.0).view(np.uint16)
    assert list(blk["qs"][0, :8]) == [127, -127, 3, -3, 1, -1, 127, -4]
    # The Q8_0 scale is the f16-rounded amax/127 and codes use 1/that f16 value.
    src2 = np.linspace(-3.3, 2.9, 32).astype(np.float32)
    b2 = oracle.quantize_q8_0(src2)
    s16 = np.float16(np.float32(3.3) / np.float32(127.0))
    assert b2["scale"][0] == s16.view(np.uint16)
    inv = np.float32(1.0) / np.float32(s16)
    y = (src2 * inv).astype(np.float64)
    q = np.clip(np.sign(y) * np.floor(np.abs(y) + 0.5), -127, 127)
    assert np.array_equal(b2["qs"][0].astype(np.int64), q.astype(np.int64))
