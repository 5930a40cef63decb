"""GPU parity of the decode FFN block (lgh_q4_ffn_residual, the fused form of
Lfm2::ffn_residual_in, crates/llm-engine/src/lfm2.rs:883-911) against the oracle.

Stage by stage, because silu's exp on the GPU and in libm may differ in the last ulp, and a
one-ulp change of h can move an ActQ8 code across a .5 tie:
  * gate/up (test hook): g and u within the GEMV tolerance of the oracle's pair GEMV of the
    oracle's rms_norm; h within 3 ulp-equivalents of silu(g) * u on the GPU's own g, u; h's
    codes and scales bit-exact to ActQ8 of the GPU's own h;
  * the whole block: hidden within the GEMV tolerance of hidden + W2 applied (oracle, AddF64)
    to exactly those codes -- the second launch is the down projection of the first's output.
"""

import numpy as np
import pytest

from llmhost_amd import q4, synth

from .conftest import assert_close, assert_close_with_flips, code_flip_bound

pytestmark = pytest.mark.gpu

SHAPES = [(1536, 8192), (96, 64), (544, 160), (2048, 256), (32, 32)]


def _mats(ctx, oracle, dim, inter, seed):
    b1 = synth.q4_blocks(seed, inter, dim)
    b3 = synth.q4_blocks(seed + 1, inter, dim)
    b2 = synth.q4_blocks(seed + 2, dim, inter)
    gpu = [q4.Q4Matrix.from_blocks(inter, dim, b1, ctx), q4.Q4Matrix.from_blocks(inter, dim, b3, ctx),
           q4.Q4Matrix.from_blocks(dim, inter, b2, ctx)]
    cpu = [oracle.Q4Matrix(inter, dim, b1), oracle.Q4Matrix(inter, dim, b3), oracle.Q4Matrix(dim, inter, b2)]
    return gpu, cpu


def _inputs(dim, seed):
    hidden = (synth.normal_f32(seed, dim) * np.float32(3.0)).astype(np.float32)
    nw = (1 + 0.2 * synth.normal_f32(seed + 1, dim)).astype(np.float32)
    return hidden, nw


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("dim,inter", SHAPES)
def test_ffn_gate_up_stage(gpu_ctx, oracle, dim, inter, per_row):
    (g1, g3, _), (c1, c3, _) = _mats(gpu_ctx, oracle, dim, inter, 10 + dim + inter)
    hidden, nw = _inputs(dim, 20 + dim)
    gpu_ctx.set_act_quant(q4.ActQuant.PerRow if per_row else q4.ActQuant.PerBlock)
    try:
        g, u, h, hq, hs = q4.ffn_gate_up(g1, g3, nw, 1e-5, hidden)
    finally:
        gpu_ctx.set_act_quant(q4.ActQuant.PerBlock)
    normed = oracle.rms_norm(hidden, nw, 1e-5)
    rg, ru = oracle.gemv_q4_pair(c1, c3, normed, per_row=per_row, threads=8)
    assert_close(g, rg, what="g")
    assert_close(u, ru, what="u")
    # h = silu(g) * u on the GPU's own g, u: four f32 roundings (exp, add, divide, multiply)
    ref_h = oracle.silu_mul(g, u).astype(np.float64)
    ulp = np.spacing(np.abs(ref_h).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(h.astype(np.float64) - ref_h) <= 4 * ulp + 1e-45)
    # h's codes: ActQ8 (PerBlock) of the GPU's h, bit-exact
    qs, sc, _ = oracle.act_quantize(h.reshape(1, -1), False)
    assert np.array_equal(hq, qs.ravel())
    assert np.array_equal(hs.view(np.uint32), sc.ravel().view(np.uint32))


def _reference_h_codes(c1, c3, nw, hidden):
    """The oracle's own h = silu(W1 n) * W3 n and its PerBlock ActQ8 codes / scales."""
    normed = hidden if nw is None else oracle_mod().rms_norm(hidden, nw, 1e-5)
    rg, ru = oracle_mod().gemv_q4_pair(c1, c3, normed, threads=8)
    h = oracle_mod().silu_mul(rg, ru)
    qs, sc, _ = oracle_mod().act_quantize(h.reshape(1, -1), False)
    return qs.ravel(), sc.ravel()


def oracle_mod():
    import oracle

    return oracle


def _check_against_composition(got, full, b2, dim, inter, hq, hs, q_ref, s_ref, what):
    """got vs the oracle's full composition: the gate tolerance plus, per element, what the h
    codes / scales that differ between the GPU's h and the oracle's h can move (silu's exp may
    differ from libm's in the last ulp, and an ulp of h can cross a .5 tie of its code)."""
    bound, flips, _ = code_flip_bound(b2, dim, inter, q_ref, s_ref, hq, hs)
    assert flips <= max(2, inter // 500), f"{what}: {flips} of {inter} h codes differ"
    # h's block scales follow h's block maxima, which move with g and u by their summation-order
    # roundings: most differ in the last bits, none by more than that
    s_ref, hs = np.asarray(s_ref, np.float64), np.asarray(hs, np.float64)
    assert np.all(np.abs(hs - s_ref) <= 1e-4 * s_ref), f"{what}: h block scales differ beyond rounding"
    assert_close_with_flips(got, full, bound, what=f"{what} ({flips} code flips)")


@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("dim,inter", SHAPES)
def test_ffn_residual_block(gpu_ctx, oracle, dim, inter, norm):
    seed = 30 + dim + inter
    (g1, g3, g2), (c1, c3, c2) = _mats(gpu_ctx, oracle, dim, inter, seed)
    b2 = synth.q4_blocks(seed + 2, dim, inter)
    hidden, nw = _inputs(dim, 40 + dim)
    nw = nw if norm else None
    _, _, _, hq, hs = q4.ffn_gate_up(g1, g3, nw, 1e-5, hidden)
    got = hidden.copy()
    q4.ffn_residual(g1, g3, g2, nw, 1e-5, got)
    ref = oracle.gemv_q4_prep(c2, hq, hs, out=hidden.copy(), add=True, threads=8)
    assert_close(got, ref, what="hidden")
    # and the whole reference composition, with an allowance only for the h codes that differ
    full = oracle.ffn_residual(c1, c3, c2, nw, 1e-5, hidden, threads=8)
    q_ref, s_ref = _reference_h_codes(c1, c3, nw, hidden)
    assert np.array_equal(oracle.gemv_q4_prep(c2, q_ref, s_ref, out=hidden.copy(), add=True, threads=8), full)
    _check_against_composition(got, full, b2, dim, inter, hq, hs, q_ref, s_ref, "vs reference composition")


def test_ffn_residual_per_row(gpu_ctx, oracle):
    """PerRow: h leaves the first launch in f32 and the down GEMV quantizes it per row."""
    dim, inter = 1536, 8192
    (g1, g3, g2), (c1, c3, c2) = _mats(gpu_ctx, oracle, dim, inter, 50)
    hidden, nw = _inputs(dim, 60)
    gpu_ctx.set_act_quant(q4.ActQuant.PerRow)
    try:
        _, _, h, _, _ = q4.ffn_gate_up(g1, g3, nw, 1e-5, hidden)
        got = hidden.copy()
        q4.ffn_residual(g1, g3, g2, nw, 1e-5, got)
    finally:
        gpu_ctx.set_act_quant(q4.ActQuant.PerBlock)
    ref = oracle.gemv_q4(c2, h, out=hidden.copy(), add=True, per_row=True, threads=8)
    assert_close(got, ref, what="hidden (PerRow)")


def test_ffn_device_path_matches_host_path(gpu_ctx, oracle):
    import torch

    dim, inter = 1536, 8192
    (g1, g3, g2), _ = _mats(gpu_ctx, oracle, dim, inter, 70)
    hidden, nw = _inputs(dim, 80)
    host = hidden.copy()
    q4.ffn_residual(g1, g3, g2, nw, 1e-5, host)
    dev = torch.from_numpy(hidden.copy()).cuda()
    q4.ffn_residual(g1, g3, g2, torch.from_numpy(nw).cuda(), 1e-5, dev)
    torch.cuda.synchronize()
    assert np.array_equal(dev.cpu().numpy(), host)


def test_ffn_shape_errors(gpu_ctx):
    b = synth.q4_blocks(1, 64, 4096)
    big1 = q4.Q4Matrix.from_blocks(64, 4096, b, gpu_ctx)
    big3 = q4.Q4Matrix.from_blocks(64, 4096, b, gpu_ctx)
    with pytest.raises(Exception, match="hidden size"):  # the fused stage alone needs dim <= 2048
        q4.ffn_gate_up(big1, big3, None, 0.0, np.zeros(4096, np.float32))
    w1 = q4.Q4Matrix.from_blocks(64, 96, synth.q4_blocks(3, 64, 96), gpu_ctx)
    w3 = q4.Q4Matrix.from_blocks(32, 96, synth.q4_blocks(4, 32, 96), gpu_ctx)
    w2 = q4.Q4Matrix.from_blocks(96, 64, synth.q4_blocks(5, 96, 64), gpu_ctx)
    with pytest.raises(Exception):
        q4.ffn_residual(w1, w3, w2, None, 0.0, np.zeros(96, np.float32))


# ---- the elementwise ops and the multi-token block ----------------------------------------
@pytest.mark.parametrize("dim,rows", [(32, 1), (1536, 1), (1536, 7), (4096, 3), (100 * 32, 2)])
def test_rms_norm_bit_exact(gpu_ctx, oracle, dim, rows):
    x = (synth.activations(dim + rows, rows, dim) * np.float32(4.0)).astype(np.float32)
    w = (1 + 0.3 * synth.normal_f32(dim, dim)).astype(np.float32)
    got = np.zeros_like(x)
    q4.rms_norm(x, w, 1e-5, got, gpu_ctx)
    assert got.tobytes() == oracle.rms_norm(x, w, 1e-5).tobytes()


def test_silu_mul_within_exp_ulp(gpu_ctx, oracle):
    g = np.concatenate([np.linspace(-40, 40, 20001), synth.normal_f32(3, 4096) * 4]).astype(np.float32)
    u = synth.normal_f32(4, g.size)
    got = g.copy()
    q4.silu_mul(got, u, gpu_ctx)
    # libm's expf and the device's expf each err by up to an ulp, so exp's two values may be two
    # ulp apart; through 1 + exp, the divide and the multiply the results stay within 4 ulp.
    ref = oracle.silu_mul(g, u).astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    err = np.abs(got.astype(np.float64) - ref) / (ulp + 1e-45)
    assert err.max() <= 4, (err.max(), g[np.argmax(err)])
    assert np.mean(got == ref.astype(np.float32)) > 0.9


def _per_op(gpu_mats, nw, hidden, t, h_out=None):
    """The block composed from the library's per-op entry points (the multi-token path's own
    sequence of launches); h_out receives h = silu(g) * u."""
    g1, g3, g2 = gpu_mats
    normed = np.zeros_like(hidden)
    if nw is not None:
        q4.rms_norm(hidden, nw, 1e-5, normed, g1.ctx)
    else:
        normed = hidden.copy()
    g = np.zeros(t * g1.n, np.float32)
    u = np.zeros(t * g1.n, np.float32)
    if t == 1:
        q4.gemv_q4_pair(g1, g3, normed, g, u)
    else:
        q4.gemm_q4(g1, normed, g, t)
        q4.gemm_q4(g3, normed, u, t)
    q4.silu_mul(g, u, g1.ctx)
    if h_out is not None:
        h_out[:] = g
    out = hidden.copy()
    (q4.gemv_q4_add(g2, g, out) if t == 1 else q4.gemm_q4_add(g2, g, out, t))
    return out


@pytest.mark.parametrize("dim,inter,t", [(1536, 8192, 1), (1536, 8192, 4), (1536, 8192, 16), (96, 64, 70),
                                         (4096, 64, 1), (544, 160, 3)])
def test_ffn_residual_matches_per_op_composition(gpu_ctx, oracle, dim, inter, t):
    """Every path of lgh_q4_ffn_residual equals the per-op composition bit for bit (the fused
    one-token launches included: same dots, same silu, same codes), and the oracle's
    composition up to the ties one ulp of exp can move."""
    seed = 90 + t + dim
    gpu, cpu = _mats(gpu_ctx, oracle, dim, inter, seed)
    b2 = synth.q4_blocks(seed + 2, dim, inter)
    hidden = (synth.activations(100 + t, t, dim) * np.float32(2.0)).astype(np.float32).ravel()
    nw = (1 + 0.2 * synth.normal_f32(101, dim)).astype(np.float32)
    got = hidden.copy()
    q4.ffn_residual(*gpu, nw, 1e-5, got, tokens=t)
    h_gpu = np.zeros(t * inter, np.float32)
    assert got.tobytes() == _per_op(gpu, nw, hidden, t, h_gpu).tobytes()
    ref = oracle.ffn_residual(*cpu, nw, 1e-5, hidden, tokens=t, threads=8)
    # the oracle's own h, as its composition forms it (lfm2.rs:861-881: the pair for one token,
    # two GEMMs for several)
    if t == 1:
        q_all, s_all = _reference_h_codes(cpu[0], cpu[1], nw, hidden)
    else:
        normed = oracle.rms_norm(hidden, nw, 1e-5)
        h_ref = oracle.silu_mul(oracle.gemm_q4(cpu[0], normed, t, threads=8),
                                oracle.gemm_q4(cpu[1], normed, t, threads=8))
        q_all, s_all, _ = oracle.act_quantize(h_ref.reshape(t, inter), False)
    q_all, s_all = q_all.reshape(t, inter), s_all.reshape(t, inter // 32)
    hq_all, hs_all, _ = oracle.act_quantize(h_gpu.reshape(t, inter), False)  # bit-exact to the device's
    for i in range(t):  # per token: the allowance for the h codes that differ from the oracle's
        row = slice(i * dim, (i + 1) * dim)
        _check_against_composition(got[row], ref[row], b2, dim, inter, hq_all[i], hs_all[i], q_all[i], s_all[i],
                                   f"token {i} vs reference composition")


def test_ffn_residual_tokens_device_path(gpu_ctx, oracle):
    import torch

    dim, inter, t = 1536, 8192, 8
    gpu, _ = _mats(gpu_ctx, oracle, dim, inter, 120)
    hidden = synth.activations(121, t, dim).ravel()
    nw = (1 + 0.2 * synth.normal_f32(122, dim)).astype(np.float32)
    host = hidden.copy()
    q4.ffn_residual(*gpu, nw, 1e-5, host, tokens=t)
    dev = torch.from_numpy(hidden.copy()).cuda()
    q4.ffn_residual(*gpu, torch.from_numpy(nw).cuda(), 1e-5, dev, tokens=t)
    torch.cuda.synchronize()
    assert np.array_equal(dev.cpu().numpy(), host)


# (dim, inter, tokens): the matrix-core batch route (5-64 tokens) and the GEMM route (65+), rows
# of an odd block count (1568 = 49 blocks: a padding block in every pair), token counts that end
# inside a 16- and a 32-token tile, the down GEMM with split K (inter 4096, 130 tokens), and rows
# longer than the fused norm covers (2080 = 65 blocks: rms_norm is written out first).
PREFILL = [(1536, 2048, 5), (1568, 2048, 37), (1536, 4096, 130), (1568, 1024, 100), (2048, 1536, 513),
           (2080, 512, 70), (96, 64, 65), (1536, 8192, 64)]


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("dim,inter,t", PREFILL)
def test_prefill_fusions_equal_op_sequence(gpu_ctx, oracle, dim, inter, t, per_row):
    """The prefill FFN block forms rms_norm(hidden) inside the gate/up activation image and
    silu(g) * u inside the down projection's image: bit for bit the op sequence it replaces
    (rms_norm; the gate/up pair on one shared activation quantization; silu_mul; the down GEMM
    added in f64), in both act-quant modes.  The same for the norm + projections entry point."""
    print(f"[prefill fusion] dim={dim} inter={inter} t={t} per_row={per_row}", flush=True)
    gpu, _ = _mats(gpu_ctx, oracle, dim, inter, 300 + dim + t)
    hidden = (synth.activations(310 + t, t, dim) * np.float32(2.0)).astype(np.float32).ravel()
    nw = (1 + 0.2 * synth.normal_f32(311 + dim, dim)).astype(np.float32)
    gpu_ctx.set_act_quant(q4.ActQuant.PerRow if per_row else q4.ActQuant.PerBlock)
    try:
        fused = hidden.copy()
        q4.ffn_residual(*gpu, nw, 1e-5, fused, tokens=t)
        normed = np.zeros_like(hidden)
        q4.rms_norm(hidden, nw, 1e-5, normed, gpu_ctx)
        g = np.zeros(t * inter, np.float32)
        u = np.zeros(t * inter, np.float32)
        q4.norm_gemv(gpu[:2], None, 1e-5, normed, [g, u], t)
        q4.silu_mul(g, u, gpu_ctx)
        seq = hidden.copy()
        q4.gemm_q4_add(gpu[2], g, seq, t)
        # norm + projections: fused vs rms_norm then the same launch without the norm
        gu_fused = [np.zeros(t * inter, np.float32), np.zeros(t * inter, np.float32)]
        q4.norm_gemv(gpu[:2], nw, 1e-5, hidden, gu_fused, t)
        g2, u2 = np.zeros(t * inter, np.float32), np.zeros(t * inter, np.float32)
        q4.norm_gemv(gpu[:2], None, 1e-5, normed, [g2, u2], t)
    finally:
        gpu_ctx.set_act_quant(q4.ActQuant.PerBlock)
    assert np.isfinite(fused).all()
    assert fused.tobytes() == seq.tobytes(), "FFN block differs from the op sequence"
    assert gu_fused[0].tobytes() == g2.tobytes() and gu_fused[1].tobytes() == u2.tobytes(), \
        "norm + projections differ from rms_norm then the projections"


# Rows of more than 128 blocks: the launch that forms the norm and the activation image loads a
# row in rounds of 128 blocks, so these cover its later rounds (one block in the last round at
# K = 4128); odd block counts cover the padding block of the last pair or quad.
@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("k,n,t", [(8288, 256, 20), (8288, 300, 70), (12320, 96, 130), (4128, 64, 5)])
def test_norm_projections_long_rows_equal_op_sequence(gpu_ctx, k, n, t, per_row):
    """norm + two projections over rows of 129-385 blocks, on the matrix-core batch route (5 and 20
    tokens) and the GEMM route (70 and 130), equal rms_norm then the projections bit for bit."""
    print(f"[norm long rows] k={k} n={n} t={t} per_row={per_row}", flush=True)
    blocks = [synth.q4_blocks(700 + k + j, n, k) for j in range(2)]
    w = [q4.Q4Matrix.from_blocks(n, k, b, gpu_ctx) for b in blocks]
    hidden = (synth.activations(710 + t, t, k) * np.float32(2.0)).astype(np.float32).ravel()
    nw = (1 + 0.2 * synth.normal_f32(711 + k, k)).astype(np.float32)
    gpu_ctx.set_act_quant(q4.ActQuant.PerRow if per_row else q4.ActQuant.PerBlock)
    try:
        normed = np.zeros_like(hidden)
        q4.rms_norm(hidden, nw, 1e-5, normed, gpu_ctx)
        fused = [np.zeros(t * n, np.float32) for _ in range(2)]
        q4.norm_gemv(w, nw, 1e-5, hidden, fused, t)
        seq = [np.zeros(t * n, np.float32) for _ in range(2)]
        q4.norm_gemv(w, None, 1e-5, normed, seq, t)
    finally:
        gpu_ctx.set_act_quant(q4.ActQuant.PerBlock)
        for m in w:
            m.free()
    for j in range(2):
        assert np.isfinite(fused[j]).all()
        assert fused[j].tobytes() == seq[j].tobytes(), f"matrix {j}"
