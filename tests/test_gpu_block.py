"""GPU parity of the attention / conv block input and output sides.

  * lgh_q4_norm_gemv: rms_norm of hidden, then 1..3 projections sharing K (Lfm2::attn_decode's
    q/k/v, crates/llm-engine/src/lfm2.rs:784-794; Lfm2::conv_update's in_proj, lfm2.rs:651-659).
    Against the oracle's rms_norm followed by its scalar-order GEMV (the reference operation
    order) within the output tolerance (1e-4 + 1e-5 |ref|), and bit for bit against the library's own op
    sequence (lgh_rms_norm, then one lgh_q4_gemm per matrix) -- the one-launch form shares one
    activation quantization and must not change a single output bit.
  * LGH_ADD_F32 (Linear::apply then ops::add_inplace, crates/llm-cpu/src/ops.rs:48-53, after
    out_proj at lfm2.rs:645, 682, 749, 857): on every M route the result equals, bit for bit,
    the same route's Assign result added to the old values in f32.
"""

import numpy as np
import pytest

from llmhost_amd import q4, synth
from llmhost_amd._ffi import LGH_ADD_F32, LGH_ADD_F64, LghError, LghShapeError

from .conftest import assert_close

pytestmark = pytest.mark.gpu

EPS = 1e-5

# (k, row counts of the 1..3 matrices): LFM2-700M attention (hidden 1536, 24 q heads and 8 kv
# heads of 64) and conv in_proj (3 * hidden), ragged and tiny rows, a K past one slice.
BLOCKS = [
    (1536, (1536, 512, 512)),
    (1536, (4608,)),
    (1536, (2048, 1536)),
    (64, (4, 36, 100)),
    (800, (33,)),
    (2048, (96, 32, 8)),
    (4096, (256, 64)),  # K > 2048: rms_norm, then one GEMM per matrix
]


def _mats(ctx, oracle, k, rows, seed):
    bl = [synth.q4_blocks(seed + j, n, k) for j, n in enumerate(rows)]
    return ([q4.Q4Matrix.from_blocks(n, k, b, ctx) for n, b in zip(rows, bl)],
            [oracle.Q4Matrix(n, k, b) for n, b in zip(rows, bl)])


def _hidden(k, tokens, seed):
    hidden = (synth.normal_f32(seed, tokens * k) * np.float32(2.5)).astype(np.float32)
    nw = (1 + 0.2 * synth.normal_f32(seed + 1, k)).astype(np.float32)
    return hidden, nw


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("norm", [True, False])
# tokens: the one-launch GEMV, the M <= 4 batch kernel, the matrix-core batch kernel on one shared
# activation image, the GEMM over all matrices in one launch (at K=4096 with K split 4 ways and
# one split-K reduce over all matrices).
@pytest.mark.parametrize("tokens", [1, 3, 16, 100])
@pytest.mark.parametrize("k,rows", BLOCKS)
def test_norm_gemv_matches_oracle_and_op_sequence(gpu_ctx, oracle, k, rows, tokens, norm, per_row):
    gw, cw = _mats(gpu_ctx, oracle, k, rows, 500 + k + sum(rows))
    hidden, nw = _hidden(k, tokens, 60 + k)
    nw = nw if norm else None
    outs = [np.full(tokens * n, np.nan, dtype=np.float32) for n in rows]
    gpu_ctx.set_act_quant(q4.ActQuant.PerRow if per_row else q4.ActQuant.PerBlock)
    try:
        q4.norm_gemv(gw, nw, EPS, hidden, outs, tokens)
        # the library's own op sequence
        normed = hidden.copy()
        if nw is not None:
            q4.rms_norm(hidden, nw, EPS, normed, gpu_ctx)
        seq = [np.zeros(tokens * n, dtype=np.float32) for n in rows]
        for w, o in zip(gw, seq):
            q4.gemm_q4(w, normed, o, tokens)
    finally:
        gpu_ctx.set_act_quant(q4.ActQuant.PerBlock)
    for j, (o, s) in enumerate(zip(outs, seq)):
        assert np.array_equal(o.view(np.uint32), s.view(np.uint32)), f"matrix {j} differs from the op sequence"
    ref_normed = hidden if nw is None else oracle.rms_norm(hidden, nw, EPS)
    for j, (o, c) in enumerate(zip(outs, cw)):
        ref = oracle.gemm_q4(c, ref_normed, tokens, per_row=per_row, kernel=oracle.KERNEL_SCALAR, threads=8)
        assert_close(o, ref.ravel(), what=f"matrix {j}")


def test_norm_gemv_device_pointers_and_add(gpu_ctx, oracle):
    import torch

    k, rows = 1536, (1536, 512, 512)
    gw, _ = _mats(gpu_ctx, oracle, k, rows, 900)
    hidden, nw = _hidden(k, 1, 901)
    y0 = [synth.normal_f32(910 + j, n) for j, n in enumerate(rows)]
    for mode in (LGH_ADD_F64, LGH_ADD_F32):
        dev = [torch.from_numpy(y.copy()).cuda() for y in y0]
        q4.norm_gemv(gw, torch.from_numpy(nw).cuda(), EPS, torch.from_numpy(hidden).cuda(), dev, 1, mode)
        gpu_ctx.sync()
        assign = [np.zeros(n, dtype=np.float32) for n in rows]
        q4.norm_gemv(gw, nw, EPS, hidden, assign, 1)
        for j, (d, a, y) in enumerate(zip(dev, assign, y0)):
            if mode == LGH_ADD_F32:
                want = y + a
            else:
                want = (y.astype(np.float64) + a.astype(np.float64)).astype(np.float32)
            assert np.array_equal(d.cpu().numpy().view(np.uint32), want.view(np.uint32)), (mode, j)


def test_norm_gemv_errors(gpu_ctx):
    a = q4.Q4Matrix.from_blocks(64, 64, synth.q4_blocks(1, 64, 64), gpu_ctx)
    b = q4.Q4Matrix.from_blocks(64, 96, synth.q4_blocks(2, 64, 96), gpu_ctx)
    h = np.zeros(64, dtype=np.float32)
    with pytest.raises(LghShapeError):
        q4.norm_gemv([a, b], None, EPS, h, [np.zeros(64, np.float32), np.zeros(64, np.float32)])
    with pytest.raises(LghShapeError):
        q4.norm_gemv([a, a, a, a], None, EPS, h, [np.zeros(64, np.float32)] * 4)
    with pytest.raises(LghError):  # unknown mode
        q4.norm_gemv([a], None, EPS, h, [np.zeros(64, np.float32)], 1, 7)
    # tokens == 0 and zero-row matrices are no-ops
    q4.norm_gemv([a], None, EPS, np.zeros(0, np.float32), [np.zeros(0, np.float32)], 0)


# One shape per route of lgh_q4_gemm_dev: the GEMV, the M <= 4 batch kernel, the matrix-core
# batch kernel, the fp6 GEMM without and with split-K, and a K past the GEMV (GEMM with M = 1).
ROUTES = [(1, 2048, 1536), (3, 1024, 1536), (16, 1024, 1536), (100, 1024, 256), (100, 1024, 1536),
          (100, 512, 10752), (1, 256, 40960)]


@pytest.mark.parametrize("m,n,k", ROUTES)
def test_add_f32_mode_every_route(gpu_ctx, m, n, k):
    w = q4.Q4Matrix.from_blocks(n, k, synth.q4_blocks(70 + m, n, k), gpu_ctx)
    x = synth.activations(71 + m, m, k)
    y0 = synth.normal_f32(72 + m, m * n).reshape(m, n)
    assign = np.zeros((m, n), dtype=np.float32)
    q4.gemm_q4(w, x, assign, m)
    got = y0.copy()
    q4.apply_add_inplace(w, x, got, m)
    assert np.array_equal(got.view(np.uint32), (y0 + assign).view(np.uint32))
    # f64 and f32 adds differ only in rounding: both within one f32 ulp of the exact sum
    f64 = y0.copy()
    q4.gemm_q4_add(w, x, f64, m)
    exact = y0.astype(np.float64) + assign.astype(np.float64)
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - exact) <= ulp) and np.all(np.abs(f64 - exact) <= 0.5 * ulp)


def test_add_f32_mode_codes_gemv(gpu_ctx):
    k, n = 1536, 640
    w = q4.Q4Matrix.from_blocks(n, k, synth.q4_blocks(80, n, k), gpu_ctx)
    x = synth.normal_f32(81, k)
    acts = q4.ActQ8.quantize(x, gpu_ctx)
    y0 = synth.normal_f32(82, n)
    assign = np.zeros(n, dtype=np.float32)
    q4.gemv_q4_prep(w, acts, assign)
    got = y0.copy()
    q4._gemv_prep(w, acts, got, LGH_ADD_F32)
    assert np.array_equal(got.view(np.uint32), (y0 + assign).view(np.uint32))


def test_seam_mirror_block_sides(gpu_ctx, oracle):
    """weights.norm_then_apply / apply_then_add_inplace on Linear objects (the seam mirror)."""
    from llmhost_amd import weights

    k, rows = 256, (256, 64, 64)
    gw, cw = _mats(gpu_ctx, oracle, k, rows, 950)
    lins = [weights.Linear(w) for w in gw]
    hidden, nw = _hidden(k, 1, 951)
    outs = [np.zeros(n, dtype=np.float32) for n in rows]
    weights.norm_then_apply(lins, nw, EPS, hidden, 1, outs)
    normed = oracle.rms_norm(hidden, nw, EPS)
    for o, c in zip(outs, cw):
        assert_close(o, oracle.gemv_q4(c, normed, kernel=oracle.KERNEL_SCALAR), what="q/k/v")
    # out_proj (256 x 64 here: the v rows back to hidden) + f32 residual
    wo = weights.Linear(gw[0])
    h2 = hidden.copy()
    weights.apply_then_add_inplace(wo, outs[0], 1, h2)
    proj = np.zeros(256, dtype=np.float32)
    wo.apply(outs[0], 1, proj)
    assert np.array_equal(h2.view(np.uint32), (hidden + proj).view(np.uint32))
    with pytest.raises(LghShapeError):
        weights.apply_then_add_inplace(wo, outs[1], 1, h2)


@pytest.mark.parametrize("tokens", [1, 2])
@pytest.mark.parametrize("n,k", [(4096, 1536), (96, 64), (130, 2048), (64, 8192), (65536, 1536)])
def test_q8_head_with_final_norm(gpu_ctx, oracle, n, k, tokens):
    """rms_norm + the Q8_0 head in one launch: bit-identical to lgh_rms_norm then lgh_q8_gemv, and
    within tolerance of the oracle's rms_norm then q8_apply (lfm2.rs:559-567).  Both matrix-size
    regimes of the kernel (whole-block lanes; half-block lanes with 8-wave workgroups for the norm),
    up to the tied head's shape."""
    from llmhost_amd import weights

    b8 = synth.q8_blocks(960 + n, n, k)
    w8 = q4.Q8Matrix.from_blocks(n, k, b8, gpu_ctx)
    hidden, nw = _hidden(k, tokens, 961 + k)
    got = np.full(tokens * n, np.nan, dtype=np.float32)
    weights.OutputHead(q8=w8).norm_apply(nw, EPS, hidden, tokens, got)
    normed = np.zeros_like(hidden)
    q4.rms_norm(hidden, nw, EPS, normed, gpu_ctx)
    seq = np.zeros(tokens * n, dtype=np.float32)
    q4.q8_apply(w8, normed, tokens, seq)
    assert np.array_equal(got.view(np.uint32), seq.view(np.uint32))
    ref = oracle.q8_apply(b8, n, k, oracle.rms_norm(hidden, nw, EPS), tokens, threads=8)
    assert_close(got, ref.ravel(), what="q8 head")
    plain = np.zeros(tokens * n, dtype=np.float32)
    q4.q8_norm_apply(w8, None, EPS, hidden, tokens, plain)
    direct = np.zeros(tokens * n, dtype=np.float32)
    q4.q8_apply(w8, hidden, tokens, direct)
    assert np.array_equal(plain.view(np.uint32), direct.view(np.uint32))
