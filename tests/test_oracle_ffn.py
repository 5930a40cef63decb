"""The oracle's decode FFN block: rms_norm (crates/llm-cpu/src/ops.rs:8-23), silu
(ops.rs:27-36) and Lfm2::ffn_residual_in (crates/llm-engine/src/lfm2.rs:883-911).

Pinned by the reference's own tests of ops.rs (:100-118), by closed forms (the sequential f64
sum of squares restated in Python, silu in float64 rounded once), and by the composition of
the oracle's already-pinned GEMV functions.
"""

import math

import numpy as np

from llmhost_amd import synth


def _rms_norm_py(x, w, eps):
    """ops.rs:8-23 in plain Python: sequential f64 sum, f64 scale, f32 products."""
    dim = len(w)
    sumsq = 0.0
    for v in x:
        sumsq += float(v) * float(v)
    scale = np.float32(1.0 / math.sqrt(sumsq * (1.0 / dim) + float(eps)))
    return (w * (x * scale)).astype(np.float32)


def test_rms_norm_reference_unit_weight(oracle):
    """rms_norm_unit_weight (ops.rs:108-118)."""
    y = oracle.rms_norm(np.array([3.0, 4.0], np.float32), np.ones(2, np.float32), 0.0)
    rms = math.sqrt((9.0 + 16.0) / 2.0)
    assert abs(y[0] - 3.0 / rms) < 1e-6 and abs(y[1] - 4.0 / rms) < 1e-6


def test_rms_norm_closed_form_bit_exact(oracle):
    rng = np.random.default_rng(5)
    for dim, rows, eps in [(32, 1, 1e-5), (96, 3, 1e-6), (1536, 2, 1e-5)]:
        x = (rng.standard_normal(dim * rows) * 3).astype(np.float32)
        w = (rng.standard_normal(dim) * 0.5 + 1).astype(np.float32)
        got = oracle.rms_norm(x, w, eps)
        ref = np.concatenate([_rms_norm_py(x[r * dim:(r + 1) * dim], w, eps) for r in range(rows)])
        assert got.tobytes() == ref.tobytes()
    # a zero row: scale = 1/sqrt(eps), output exactly 0
    z = oracle.rms_norm(np.zeros(64, np.float32), np.ones(64, np.float32), 1e-5)
    assert not z.any()


def test_silu_reference_signs_and_rounding(oracle):
    """silu_at_zero_is_zero (ops.rs:100-106), then against float64 silu: the f32 formula
    x / (1 + exp(-x)) rounds three times (exp, add, divide), so it stays within 3 ulp."""
    s = oracle.silu_mul(np.array([0.0, 2.0, -2.0], np.float32), np.ones(3, np.float32))
    assert abs(s[0]) < 1e-7 and s[1] > 1.0 and s[2] < 0.0
    g = np.linspace(-30, 30, 4001).astype(np.float32)
    u = np.ones_like(g)
    got = oracle.silu_mul(g, u).astype(np.float64)
    exact = g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - exact) <= 3 * ulp + 1e-45)
    # the product with u is one more f32 rounding: (silu(g) * u)
    u2 = np.linspace(-3, 3, g.size).astype(np.float32)
    assert np.array_equal(oracle.silu_mul(g, u2), (oracle.silu_mul(g, u) * u2).astype(np.float32))


def test_ffn_residual_is_the_reference_composition(oracle):
    dim, inter = 96, 64
    w1 = oracle.Q4Matrix(inter, dim, synth.q4_blocks(1, inter, dim))
    w3 = oracle.Q4Matrix(inter, dim, synth.q4_blocks(2, inter, dim))
    w2 = oracle.Q4Matrix(dim, inter, synth.q4_blocks(3, dim, inter))
    hidden = synth.normal_f32(4, dim)
    nw = (1 + 0.1 * synth.normal_f32(5, dim)).astype(np.float32)
    for per_row in (False, True):
        got = oracle.ffn_residual(w1, w3, w2, nw, 1e-5, hidden, per_row=per_row, threads=2)
        normed = oracle.rms_norm(hidden, nw, 1e-5)
        g, u = oracle.gemv_q4_pair(w1, w3, normed, per_row=per_row)
        h = oracle.silu_mul(g, u)
        ref = oracle.gemv_q4(w2, h, out=hidden.copy(), add=True, per_row=per_row)
        assert got.tobytes() == ref.tobytes()
    # norm_w None: the GEMVs read hidden itself
    got = oracle.ffn_residual(w1, w3, w2, None, 0.0, hidden)
    g, u = oracle.gemv_q4_pair(w1, w3, hidden)
    ref = oracle.gemv_q4(w2, oracle.silu_mul(g, u), out=hidden.copy(), add=True)
    assert got.tobytes() == ref.tobytes()


def test_ffn_residual_tokens_is_the_reference_composition(oracle):
    """Lfm2::ffn_residual (lfm2.rs:861-881): rms_norm per row, two GEMMs (apply_pair with
    tokens > 1), silu * u, gemm_q4_add."""
    dim, inter, t = 64, 96, 5
    w1 = oracle.Q4Matrix(inter, dim, synth.q4_blocks(11, inter, dim))
    w3 = oracle.Q4Matrix(inter, dim, synth.q4_blocks(12, inter, dim))
    w2 = oracle.Q4Matrix(dim, inter, synth.q4_blocks(13, dim, inter))
    hidden = synth.activations(14, t, dim)
    nw = (1 + 0.1 * synth.normal_f32(15, dim)).astype(np.float32)
    got = oracle.ffn_residual(w1, w3, w2, nw, 1e-5, hidden, tokens=t)
    normed = oracle.rms_norm(hidden, nw, 1e-5)
    g = oracle.gemm_q4(w1, normed, t)
    u = oracle.gemm_q4(w3, normed, t)
    h = oracle.silu_mul(g, u)
    ref = oracle.gemm_q4(w2, h, t, out=hidden.copy(), add=True)
    assert got.tobytes() == ref.tobytes()
