"""GPU parity: libllm_gpu_hip.so (through the C ABI) against the CPU oracle.

Bar: bit-exact for integer work (activation codes / scales / sums, per-block
dots, weight repack and quantize), |gpu - cpu| <= 1e-4 + 1e-5 |cpu| for fp32
outputs, against the oracle's scalar kernel (the reference operation order)
and its VNNI kernel (the production CPU path) on identical seeded inputs.
"""

import numpy as np
import pytest

from llmhost_amd import _ffi, formats, q4, synth
from llmhost_amd.formats import BLOCK_Q4

from .conftest import assert_close, assert_close_with_flips, q8_exact_terms, summation_allowance

pytestmark = pytest.mark.gpu


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- bit-exact integer work ---------------------------------------------------------
@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("m,k", [(1, 32), (1, 1536), (3, 8192), (17, 2048), (2, 10752)])
def test_act_quant_bit_exact(gpu_ctx, oracle, per_row, m, k):
    x = synth.activations(1000 + k + m, m, k) * np.float32(2.5)
    x[0, :32] = 0.0                     # zero block
    if k >= 64:
        x[-1, 32:36] = [127.0, 2.5, -2.5, 0.5]  # exact ties after scaling by 1/1
    x = _f32(x)
    act = (q4.ActQ8.quantize_row if per_row else q4.ActQ8.quantize)(x, gpu_ctx)
    qs, sc, su = oracle.act_quantize(x, per_row)
    assert np.array_equal(act.scales.view(np.uint32), sc.view(np.uint32))
    assert np.array_equal(act.qs, qs)
    assert np.array_equal(act.sums, su)


def test_act_quant_ties(gpu_ctx, oracle):
    x = np.zeros((1, 64), dtype=np.float32)
    x[0, :8] = [127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -1.5, 3.5]
    act = q4.ActQ8.quantize(x, gpu_ctx)
    assert list(act.qs[0, :8]) == [127, 3, -3, 1, -1, 127, -2, 4]
    assert act.scales[0, 0] == 1.0 and act.scales[0, 1] == 0.0


def _nan_blocks(k, seed):
    """x with NaN edge blocks: Rust's amax folds |v| into 0.0 with f32::max, which skips NaN,
    so an all-NaN block has scale 0, and `NaN as i8` is 0."""
    x = synth.normal_f32(seed, k) * np.float32(3.0)
    x[:32] = np.nan                       # all NaN: amax 0, scale 0, codes 0
    x[32:64:3] = np.nan                   # some NaN: the others set amax
    x[96:128] = 0.0
    x[100] = np.float32(1e-40)            # denormal amax: 1/scale overflows
    x[128:160:5] = -np.inf                # inf amax: scale inf, inv 0, codes NaN -> 0
    return _f32(x)


@pytest.mark.parametrize("per_row", [False, True])
def test_act_quant_nan_and_inf_blocks(gpu_ctx, oracle, per_row):
    x = np.stack([_nan_blocks(256, 7), _nan_blocks(256, 6)[::-1].copy()])
    x[1, 128:160] = 0.25  # the second row finite apart from NaN
    act = (q4.ActQ8.quantize_row if per_row else q4.ActQ8.quantize)(_f32(x), gpu_ctx)
    qs, sc, su = oracle.act_quantize(_f32(x), per_row)
    assert np.array_equal(act.scales.view(np.uint32), sc.view(np.uint32))
    assert np.array_equal(act.qs, qs)
    assert np.array_equal(act.sums, su)
    if not per_row:
        assert act.scales[0, 0] == 0.0 and not act.qs[0, :32].any()
        assert act.scales[0, 4] == np.inf  # inf / 127


def test_gemv_nan_blocks_match_oracle(gpu_ctx, oracle):
    """The GEMV's in-kernel quantizer on NaN blocks (no inf: 0 * inf would make the row NaN)."""
    n, k = 96, 1536
    x = _nan_blocks(k, 8)
    x[128:160] = 0.5
    b = synth.q4_blocks(9, n, k)
    y = np.zeros(n, np.float32)
    q4.gemv_q4(q4.Q4Matrix.from_blocks(n, k, b, gpu_ctx), x, y)
    ref = oracle.gemv_q4(oracle.Q4Matrix(n, k, b), x)
    assert np.isfinite(ref).all()
    assert_close(y, ref)


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("m", [2, 20, 70, 130])
def test_gemm_special_blocks_match_oracle(gpu_ctx, oracle, per_row, m):
    """Every token-count route's activation quantizer (in the batch kernel, the MMA image, the
    GEMM's fp6 image) on NaN blocks, a denormal block max (1/scale overflows: the reference's own
    rounding path), exact .5 ties and zero blocks, against the oracle's GEMM.  No inf: 0 * inf
    would make a row NaN."""
    n, k = 97, 512
    rows = []
    for t in range(m):
        x = _nan_blocks(k, 60 + t)
        x[128:160] = 0.5 * (t % 3)        # zero block for every third token
        x[160:168] = [127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -1.5, 3.5]  # ties (amax 127: scale 1)
        x[168:192] = 0.0
        rows.append(x if t % 2 == 0 else x[::-1].copy())
    x = _f32(np.stack(rows))
    b = synth.q4_blocks(61 + m, n, k)
    gpu_ctx.set_act_quant(q4.ActQuant.PerRow if per_row else q4.ActQuant.PerBlock)
    try:
        got = np.zeros((m, n), dtype=np.float32)
        q4.gemm_q4(q4.Q4Matrix.from_blocks(n, k, b, gpu_ctx), x, got, m)
    finally:
        gpu_ctx.set_act_quant(q4.ActQuant.PerBlock)
    ref = oracle.gemm_q4(oracle.Q4Matrix(n, k, b), x, m, per_row=per_row, threads=8)
    assert np.isfinite(ref).all()
    assert_close(got, ref, what=f"m={m}")


# ---- gemv_q4_prep and the device act-quant ---------------------------------------------
@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("n,k", [(8192, 1536), (1536, 8192), (70, 96), (33, 32 * 33), (5, 32768), (300, 65536),
                                 (40, 32800)])
def test_gemv_prep_matches_oracle(gpu_ctx, oracle, n, k, per_row):
    """gemv_q4_prep / _add (gemv_q4.rs:366-393) on the device's ActQ8 of x (bit-exact to the
    oracle's), against the oracle's gemv_q4_prep on the same codes."""
    b = synth.q4_blocks(40 + n + k, n, k)
    wg, wc = q4.Q4Matrix.from_blocks(n, k, b, gpu_ctx), oracle.Q4Matrix(n, k, b)
    x = synth.normal_f32(41 + k, k)
    acts = (q4.ActQ8.quantize_row if per_row else q4.ActQ8.quantize)(x.reshape(1, -1), gpu_ctx)
    qs, sc, _ = oracle.act_quantize(x.reshape(1, -1), per_row)
    assert np.array_equal(acts.qs, qs) and np.array_equal(acts.scales.view(np.uint32), sc.view(np.uint32))
    got = np.zeros(n, np.float32)
    q4.gemv_q4_prep(wg, acts, got)
    assert_close(got, oracle.gemv_q4_prep(wc, qs, sc, threads=8), what="prep")
    base = synth.normal_f32(42, n)
    got = base.copy()
    q4.gemv_q4_prep_add(wg, acts, got)
    assert_close(got, oracle.gemv_q4_prep(wc, qs, sc, out=base.copy(), add=True, threads=8), what="prep_add")
    wg.free()


@pytest.mark.parametrize("per_row", [False, True])
def test_device_act_quant_and_prep_equal_the_gemv(gpu_ctx, per_row):
    """lgh_act_quant_dev equals the host hook bit for bit, and the prepared-activation GEMV on
    its codes equals the GEMV that quantizes x itself, bit for bit (same codes, same kernel)."""
    import torch

    n, k, m = 1536, 8192, 3
    x = synth.activations(43, m, k)
    mode = q4.ActQuant.PerRow if per_row else q4.ActQuant.PerBlock
    host = (q4.ActQ8.quantize_row if per_row else q4.ActQ8.quantize)(x, gpu_ctx)
    dev = (q4.ActQ8.quantize_row if per_row else q4.ActQ8.quantize)(torch.from_numpy(x).cuda(), gpu_ctx)
    torch.cuda.synchronize()
    assert np.array_equal(dev.qs.cpu().numpy(), host.qs)
    assert np.array_equal(dev.scales.cpu().numpy().view(np.uint32), host.scales.view(np.uint32))
    assert np.array_equal(dev.sums.cpu().numpy(), host.sums)
    w = q4.Q4Matrix.from_blocks(n, k, synth.q4_blocks(44, n, k), gpu_ctx)
    y_prep = torch.zeros(n, device="cuda")
    y_gemv = torch.zeros(n, device="cuda")
    row = q4.ActQ8(dev.qs[1].contiguous(), dev.scales[1].contiguous(), dev.sums[1].contiguous())
    q4.gemv_q4_prep(w, row, y_prep)
    gpu_ctx.set_act_quant(mode)
    try:
        q4.gemv_q4(w, torch.from_numpy(x[1].copy()).cuda(), y_gemv)
    finally:
        gpu_ctx.set_act_quant(q4.ActQuant.PerBlock)
    torch.cuda.synchronize()
    assert torch.equal(y_prep, y_gemv)
    w.free()


def test_gemv_prep_errors(gpu_ctx):
    import torch

    w = q4.Q4Matrix.from_blocks(64, 96, synth.q4_blocks(45, 64, 96), gpu_ctx)
    acts = q4.ActQ8.quantize(synth.normal_f32(46, 96).reshape(1, -1), gpu_ctx)
    with pytest.raises(q4.LghShapeError):
        q4.gemv_q4_prep(w, q4.ActQ8(acts.qs[:, :64], acts.scales[:, :2], acts.sums), np.zeros(64, np.float32))
    qd = torch.zeros(97, dtype=torch.int8, device="cuda")
    sd = torch.zeros(3, dtype=torch.float32, device="cuda")
    y = torch.zeros(64, device="cuda")
    with pytest.raises(q4.LghError, match="aligned"):  # codes one byte past a 16-byte boundary
        q4.gemv_q4_prep(w, q4.ActQ8(qd[1:], sd, None), y)
    w.free()


def _pattern_block(seed):
    i = np.arange(32)
    w = (((i * 17 + seed) % 21) - 10).astype(np.float32) * np.float32(0.25)
    a = (((i * 9 + seed) % 25) - 12).astype(np.int8)
    return w, a


def test_q4_block_dots_bit_exact(gpu_ctx, oracle):
    # the reference's pattern_block seeds 0..15 (gemv_q4.rs:1080-1102) ...
    blocks, acts = [], []
    for seed in range(16):
        w, a = _pattern_block(seed)
        blocks.append(oracle.quantize_q4(w)[0])
        acts.append(a)
    # ... plus random blocks, extremes and every nibble value
    rng = np.random.default_rng(1)
    rb = synth.q4_blocks(77, 256, 32)
    rb["qs"][0] = 0x88
    rb["qs"][1] = 0x77
    blocks.extend(rb)
    for b in range(256):
        a = rng.integers(-127, 128, 32, dtype=np.int8)
        if b in (0, 1):
            a[:] = -127
        acts.append(a)
    blocks = np.array(blocks, dtype=BLOCK_Q4)
    acts = np.stack(acts)
    got = q4.q4_block_dots(blocks, acts, gpu_ctx)
    ref = np.array([oracle.dot_q4_q8(blocks[i], acts[i]) for i in range(len(blocks))])
    assert np.array_equal(got, ref)


def test_q8_block_dots_bit_exact(gpu_ctx, oracle):
    blocks = synth.q8_blocks(5, 200, 32)
    blocks["qs"][0] = -127
    rng = np.random.default_rng(2)
    acts = rng.integers(-127, 128, (200, 32), dtype=np.int8)
    acts[0] = -127
    got = q4.q8_block_dots(blocks, acts, gpu_ctx)
    ref = np.array([oracle.dot_q8_q8(blocks[i], acts[i]) for i in range(200)])
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("n,k,m", [(48, 64, 40), (17, 96, 5), (70, 256, 33)])
def test_mfma_block_dots_bit_exact(gpu_ctx, oracle, n, k, m):
    blocks = synth.q4_blocks(300 + n, n, k)
    qs = np.random.default_rng(n).integers(-127, 128, (m, k), dtype=np.int8)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    got = q4.q4_mfma_block_dots(w, qs, m)
    bpr = k // 32
    ref = np.zeros((m, n, bpr), dtype=np.int32)
    for t in range(m):
        for r in range(n):
            for b in range(bpr):
                ref[t, r, b] = oracle.dot_q4_q8(blocks[r * bpr + b], qs[t, b * 32:(b + 1) * 32])
    assert np.array_equal(got, ref)


def test_mfma_block_dots_extremes(gpu_ctx, oracle):
    """Largest block dots: nibbles -8 / 7 against activations -127 / 127 (|dot| = 32512),
    plus every h/l split boundary of the activation codes (q = 16h + l)."""
    n, k, m = 32, 64, 34
    nib = np.where((np.arange(n) % 2 == 0)[:, None], -8, 7) * np.ones((1, k), dtype=np.int8)
    nib[3, ::3] = 0
    nib = nib.astype(np.int8)
    blocks = formats.q4_from_nibbles(nib.reshape(-1, 32), np.full(n * k // 32, 0x3C00, dtype=np.uint16))
    qs = np.empty((m, k), dtype=np.int8)
    qs[0], qs[1] = -127, 127
    qs[2:] = ((np.arange((m - 2) * k) % 255) - 127).reshape(m - 2, k).astype(np.int8)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    got = q4.q4_mfma_block_dots(w, qs, m)
    ref = np.einsum("rbe,tbe->trb", nib.reshape(n, k // 32, 32).astype(np.int64),
                    qs.reshape(m, k // 32, 32).astype(np.int64)).astype(np.int32)
    assert np.abs(ref).max() == 32512
    assert np.array_equal(got, ref)
    for r in range(n):
        for b in range(k // 32):
            assert ref[5, r, b] == oracle.dot_q4_q8(blocks[r * (k // 32) + b], qs[5, b * 32:(b + 1) * 32])


def test_upload_download_roundtrip(gpu_ctx):
    blocks = synth.q4_blocks(9, 33, 160)
    w = q4.Q4Matrix.from_blocks(33, 160, blocks, gpu_ctx)
    assert w.blocks().tobytes() == blocks.tobytes()
    b8 = synth.q8_blocks(10, 21, 96)
    w8 = q4.Q8Matrix.from_blocks(21, 96, b8, gpu_ctx)
    assert w8.blocks().tobytes() == b8.tobytes()


def test_device_quantizers_bit_exact(gpu_ctx, oracle):
    n, k = 45, 224
    wf = synth.activations(12, n, k) * np.float32(0.7)
    wf[0, :32] = 0.0
    wf[1, :8] = [8.0, -8.0, 2.5, -2.5, 0.5, -0.5, 1.5, -7.5]
    wf = _f32(wf)
    assert q4.Q4Matrix.from_f32(wf, n, k, gpu_ctx).blocks().tobytes() == oracle.quantize_q4(wf).tobytes()
    assert q4.Q8Matrix.from_f32(wf, n, k, gpu_ctx).blocks().tobytes() == oracle.quantize_q8_0(wf).tobytes()


# ---- GEMV -----------------------------------------------------------------------------
GEMV_SHAPES = [(17, 64), (128, 64), (1536, 1536), (8192, 1536), (1536, 8192), (2048, 1536),
               (1000, 96), (64, 10752), (5, 32), (3, 2080), (4, 65536)]


@pytest.mark.parametrize("n,k", GEMV_SHAPES)
def test_gemv_matches_oracle(gpu_ctx, oracle, n, k):
    blocks = synth.q4_blocks(10 * n + k, n, k)
    x = synth.normal_f32(20 * n + k, k)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    got = np.zeros(n, dtype=np.float32)
    q4.gemv_q4(w, x, got)
    mat = oracle.Q4Matrix(n, k, blocks)
    assert_close(got, oracle.gemv_q4(mat, x, kernel=oracle.KERNEL_SCALAR, threads=8), what="vs scalar")
    assert_close(got, oracle.gemv_q4(mat, x, kernel=oracle.KERNEL_VNNI, threads=8), what="vs vnni")


def test_gemv_reference_formula_inputs(gpu_ctx, oracle):
    """gemv_kernels_agree / packed_gemv_matches_block_dots inputs (gemv_q4.rs:1104-1249)."""
    for n, k, (wm, wmod, wo, ws), (xm, xmod, xo, xs) in [
            (17, 64, (13, 19, 9, 0.15), (7, 15, 7, 0.2)), (128, 64, (3, 17, 8, 0.1), (5, 11, 5, 0.2))]:
        w = ((((np.arange(n * k) * wm) % wmod) - wo).astype(np.float32) * np.float32(ws)).astype(np.float32)
        x = ((((np.arange(k) * xm) % xmod) - xo).astype(np.float32) * np.float32(xs)).astype(np.float32)
        mat = oracle.Q4Matrix.from_f32(w, n, k)
        gw = q4.Q4Matrix.from_f32(w, n, k, gpu_ctx)
        got = np.zeros(n, dtype=np.float32)
        q4.gemv_q4(gw, x, got)
        assert_close(got, oracle.gemv_q4(mat, x, kernel=oracle.KERNEL_SCALAR), what=f"n={n}")


def test_gemv_add_f64(gpu_ctx, oracle):
    n, k = 1536, 8192
    blocks = synth.q4_blocks(5, n, k)
    x = synth.normal_f32(6, k)
    y0 = synth.normal_f32(7, n) * np.float32(100.0)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    got = y0.copy()
    q4.gemv_q4_add(w, x, got)
    ref = oracle.gemv_q4(oracle.Q4Matrix(n, k, blocks), x, out=y0.copy(), add=True, threads=8)
    assert_close(got, ref, what="add_f64")
    # the epilogue is exactly f32(f64(dst) + f64(W x)) of this kernel's own W x
    gx = np.zeros(n, dtype=np.float32)
    q4.gemv_q4(w, x, gx)
    assert np.array_equal(got, (y0.astype(np.float64) + gx.astype(np.float64)).astype(np.float32))


def test_gemv_per_row(gpu_ctx, oracle):
    n, k = 2048, 1536
    blocks = synth.q4_blocks(15, n, k)
    x = synth.normal_f32(16, k)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    gpu_ctx.set_act_quant(q4.ActQuant.PerRow)
    try:
        got = np.zeros(n, dtype=np.float32)
        q4.gemv_q4(w, x, got)
    finally:
        gpu_ctx.set_act_quant(q4.ActQuant.PerBlock)
    assert_close(got, oracle.gemv_q4(oracle.Q4Matrix(n, k, blocks), x, per_row=True, threads=8), what="per row")


def test_gemv_pair(gpu_ctx, oracle):
    n, k = 8192, 1536
    bg, bu = synth.q4_blocks(41, n, k), synth.q4_blocks(42, n, k)
    x = synth.normal_f32(43, k)
    wg, wu = q4.Q4Matrix.from_blocks(n, k, bg, gpu_ctx), q4.Q4Matrix.from_blocks(n, k, bu, gpu_ctx)
    og, ou = np.zeros(n, dtype=np.float32), np.zeros(n, dtype=np.float32)
    q4.gemv_q4_pair(wg, wu, x, og, ou)
    rg, ru = oracle.gemv_q4_pair(oracle.Q4Matrix(n, k, bg), oracle.Q4Matrix(n, k, bu), x, threads=8)
    assert_close(og, rg, what="gate")
    assert_close(ou, ru, what="up")
    # pair == two single GEMVs on the GPU
    sg = np.zeros(n, dtype=np.float32)
    q4.gemv_q4(wg, x, sg)
    assert np.array_equal(og, sg)


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("n,k", [(8192, 16384), (16384, 8192), (4096, 8192)])
def test_gemv_long_rows_at_large_n(gpu_ctx, oracle, n, k, per_row):
    """The plans for long rows at large N: more rows per workgroup (K=8192), and past ~12M
    re-quantized elements (K=16384, N=8192) x quantized once then the codes GEMV.
    Assign and AddF64, both act-quant modes."""
    blocks = synth.q4_blocks(n + k, n, k)
    x = synth.normal_f32(n + 2, k)
    y0 = synth.normal_f32(n + 3, n)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    mat = oracle.Q4Matrix(n, k, blocks)
    gpu_ctx.set_act_quant(q4.ActQuant.PerRow if per_row else q4.ActQuant.PerBlock)
    try:
        got = np.zeros(n, dtype=np.float32)
        q4.gemv_q4(w, x, got)
        add = y0.copy()
        q4.gemv_q4_add(w, x, add)
    finally:
        gpu_ctx.set_act_quant(q4.ActQuant.PerBlock)
    assert_close(got, oracle.gemv_q4(mat, x, per_row=per_row, threads=8), what="assign")
    assert_close(add, oracle.gemv_q4(mat, x, out=y0.copy(), add=True, per_row=per_row, threads=8), what="add")
    w.free()


def test_gemv_pair_long_rows_equals_two_gemvs(gpu_ctx, oracle):
    """A pair at K=16384 takes the quantize-once route, each single GEMV the in-kernel one:
    the codes are the same, so the results are bit-identical."""
    n, k = 4096, 16384
    bg, bu = synth.q4_blocks(51, n, k), synth.q4_blocks(52, n, k)
    x = synth.normal_f32(53, k)
    wg, wu = q4.Q4Matrix.from_blocks(n, k, bg, gpu_ctx), q4.Q4Matrix.from_blocks(n, k, bu, gpu_ctx)
    og, ou = np.zeros(n, dtype=np.float32), np.zeros(n, dtype=np.float32)
    q4.gemv_q4_pair(wg, wu, x, og, ou)
    rg, ru = oracle.gemv_q4_pair(oracle.Q4Matrix(n, k, bg), oracle.Q4Matrix(n, k, bu), x, threads=8)
    assert_close(og, rg, what="gate")
    assert_close(ou, ru, what="up")
    sg, su = np.zeros(n, dtype=np.float32), np.zeros(n, dtype=np.float32)
    q4.gemv_q4(wg, x, sg)
    q4.gemv_q4(wu, x, su)
    assert np.array_equal(og, sg) and np.array_equal(ou, su)
    wg.free()
    wu.free()


# ---- GEMM -----------------------------------------------------------------------------
@pytest.mark.parametrize("m,n,k", [(2, 48, 64), (4, 8192, 2048), (16, 512, 2048), (20, 48, 64),
                                   (40, 48, 64), (64, 1000, 2048), (100, 257, 320), (512, 256, 2048),
                                   (130, 2048, 10752), (33, 70, 96), (257, 130, 1056)])
def test_gemm_matches_oracle(gpu_ctx, oracle, m, n, k):
    blocks = synth.q4_blocks(n + 7 * k, n, k)
    x = synth.activations(m + 3 * k, m, k)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    got = np.zeros((m, n), dtype=np.float32)
    q4.gemm_q4(w, x, got, m)
    mat = oracle.Q4Matrix(n, k, blocks)
    assert_close(got, oracle.gemm_q4(mat, x, m, kernel=oracle.KERNEL_SCALAR, threads=8), what="vs scalar")
    assert_close(got, oracle.gemm_q4(mat, x, m, kernel=oracle.KERNEL_VNNI, threads=8), what="vs vnni")


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("m,n,k", [(2, 37, 32), (3, 131, 96), (4, 260, 544), (5, 77, 2048), (8, 130, 3072),
                                   (9, 67, 1024), (16, 301, 2048), (4, 129, 4096), (3, 45, 8192),
                                   (8, 64, 4096), (16, 33, 1536), (6, 50, 256), (12, 40, 416),
                                   (24, 129, 4096), (48, 77, 1056), (64, 40, 8192), (33, 16, 544),
                                   (40, 77, 1568), (33, 8192, 2048), (48, 130, 8192), (35, 8191, 1536),
                                   (45, 8193, 1536), (16, 1536, 8192), (7, 100, 16384), (13, 200, 4128),
                                   (11, 300, 6816), (64, 300, 8000), (56, 130, 7168)])
def test_small_batch_gemv_path(gpu_ctx, oracle, per_row, m, n, k):
    """2 <= m <= 64: the dot4 batch kernel (m <= 4) and the MFMA batch kernel (1 to 4 token
    tiles of 16, 1/2/4/8 K slices, 8-block chunks, and 4-block chunks for three token tiles over
    rows of >= 48 blocks and <= 8192 rows, ragged chunk tails; one or four token tiles over 3-16
    chunks per wave, uneven slices and a partial last chunk included, with the next chunk's
    weights in flight), Assign and AddF64."""
    blocks = synth.q4_blocks(m + n + k, n, k)
    x = synth.activations(m * 7 + k, m, k)
    y0 = synth.activations(n + 5, m, n)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    mat = oracle.Q4Matrix(n, k, blocks)
    gpu_ctx.set_act_quant(q4.ActQuant.PerRow if per_row else q4.ActQuant.PerBlock)
    try:
        got = np.zeros((m, n), dtype=np.float32)
        q4.gemm_q4(w, x, got, m)
        added = y0.copy()
        q4.gemm_q4_add(w, x, added, m)
    finally:
        gpu_ctx.set_act_quant(q4.ActQuant.PerBlock)
    assert_close(got, oracle.gemm_q4(mat, x, m, per_row=per_row, threads=8), what="batch assign")
    assert_close(added, oracle.gemm_q4(mat, x, m, out=y0.copy(), add=True, per_row=per_row, threads=8),
                 what="batch add")


def test_gemm_matches_per_token_gemv_reference_inputs(gpu_ctx, oracle):
    """gemm_matches_per_token_gemv (gemv_q4.rs:1167-1195) and the AMX test (amx.rs:526-557)."""
    for n, k, m in [(48, 64, 20), (48, 64, 40)]:
        w = ((((np.arange(n * k) * 3) % 17) - 8).astype(np.float32) * np.float32(0.1)).astype(np.float32)
        x = ((((np.arange(m * k) * 5) % 11) - 5).astype(np.float32) * np.float32(0.2)).astype(np.float32)
        gw = q4.Q4Matrix.from_f32(w, n, k, gpu_ctx)
        gemm = np.zeros(m * n, dtype=np.float32)
        q4.gemm_q4(gw, x, gemm, m)
        gemv = np.zeros(m * n, dtype=np.float32)
        for t in range(m):
            out = np.zeros(n, dtype=np.float32)
            q4.gemv_q4(gw, np.ascontiguousarray(x[t * k:(t + 1) * k]), out)
            gemv[t * n:(t + 1) * n] = out
        assert np.all(np.abs(gemm - gemv) <= 1e-5 * (1 + np.abs(gemv)))
        assert_close(gemm.reshape(m, n), oracle.gemm_q4(oracle.Q4Matrix.from_f32(w, n, k), x, m), what="oracle")


@pytest.mark.parametrize("per_row", [False, True])
def test_gemm_add_and_per_row(gpu_ctx, oracle, per_row):
    m, n, k = 64, 768, 1024
    blocks = synth.q4_blocks(51, n, k)
    x = synth.activations(52, m, k)
    y0 = synth.activations(53, m, n)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    gpu_ctx.set_act_quant(q4.ActQuant.PerRow if per_row else q4.ActQuant.PerBlock)
    try:
        got = y0.copy()
        q4.gemm_q4_add(w, x, got, m)
    finally:
        gpu_ctx.set_act_quant(q4.ActQuant.PerBlock)
    ref = oracle.gemm_q4(oracle.Q4Matrix(n, k, blocks), x, m, out=y0.copy(), add=True, per_row=per_row,
                         threads=8)
    assert_close(got, ref, what="gemm add")


# ---- Q8_0 GEMV ---------------------------------------------------------------------------
@pytest.mark.parametrize("n,k,tokens", [(1536, 1536, 1), (77, 256, 3), (4096, 1536, 2), (65536, 1536, 1),
                                         (300, 4096, 2), (70, 8192, 1), (33, 16384, 1), (20, 32768, 2),
                                         (5, 32, 3), (1, 64, 1), (130, 96, 4), (16384, 4096, 1),
                                         (16400, 2080, 2)])
def test_q8_gemv_matches_oracle(gpu_ctx, oracle, n, k, tokens):
    """Every plan of the Q8_0 GEMV: one K slice (1..4 blocks per lane), 2 / 4 / 8 / 16 slices
    (2 slices of 4 blocks per lane: rows of 65-128 blocks at N >= 16384, a tied head of hidden
    2080-4096), rows not a multiple of 4, several tokens (grid.y), the N=65536 head."""
    blocks = synth.q8_blocks(n + k, n, k)
    x = synth.activations(tokens + k, tokens, k)
    w = q4.Q8Matrix.from_blocks(n, k, blocks, gpu_ctx)
    got = np.zeros((tokens, n) if tokens > 1 else n, dtype=np.float32)
    q4.q8_apply(w, x, tokens, got)
    assert_close(got, oracle.q8_apply(blocks, n, k, x, tokens, threads=8), what="q8")


@pytest.mark.parametrize("n,k,tokens", [(2, 32 * 1025, 1), (70, 65536, 2), (300, 100000 // 32 * 32, 1)])
def test_q8_gemv_long_rows(gpu_ctx, oracle, n, k, tokens):
    """K past one launch's 32768: K ranges of 32768 whose partial sums add in f32 (q8_apply has no
    K limit, weights.rs:194-227).  With Q8 codes of +-127 over 2048+ blocks the partial sums of
    the f32 accumulation reach ~10^2, so summation order alone moves a result by more than the
    1e-4 gate where it cancels to a small value: the device and the oracle are both held to the
    exact value (f64; every term is exact) within the gate plus the f32 summation allowance."""
    blocks = synth.q8_blocks(9 + k, n, k)
    x = synth.activations(10 + k, tokens, k)
    nw = (1 + 0.1 * synth.normal_f32(11 + k, k)).astype(np.float32)
    w = q4.Q8Matrix.from_blocks(n, k, blocks, gpu_ctx)
    got = np.zeros(tokens * n, np.float32)
    q4.q8_apply(w, x, tokens, got)
    normed = np.zeros(tokens * n, np.float32)
    q4.q8_norm_apply(w, nw, 1e-5, x, tokens, normed)  # the norm as its own launch before the ranges
    for what, dev, xin in (("q8 long rows", got, x), ("norm + q8 long rows", normed, oracle.rms_norm(x, nw, 1e-5))):
        qs, sa, _ = oracle.act_quantize(xin.reshape(tokens, k), False)
        exact, R = q8_exact_terms(blocks, n, k, qs, sa)
        allow = summation_allowance(R, k // 32).ravel()
        ref = oracle.q8_apply(blocks, n, k, xin, tokens, threads=8).ravel()
        assert_close_with_flips(ref, exact.ravel(), allow, what=f"oracle vs exact, {what}")
        assert_close_with_flips(dev, exact.ravel(), allow, what=f"device vs exact, {what}")
    w.free()


def test_q8_gemv_more_tokens_than_one_grid(gpu_ctx, oracle):
    """More than 65535 tokens: further launches over the token rows (grid.y holds 65535)."""
    n, k, tokens = 6, 64, 70001
    blocks = synth.q8_blocks(12, n, k)
    x = synth.activations(13, tokens, k)
    w = q4.Q8Matrix.from_blocks(n, k, blocks, gpu_ctx)
    got = np.zeros((tokens, n), np.float32)
    q4.q8_apply(w, x, tokens, got)
    assert_close(got, oracle.q8_apply(blocks, n, k, x, tokens, threads=8), what="q8 many tokens")
    w.free()


# ---- error behaviour --------------------------------------------------------------------------
def test_shape_errors(gpu_ctx):
    with pytest.raises(q4.LghShapeError):
        q4.Q4Matrix.from_blocks(4, 48, np.zeros(6, dtype=BLOCK_Q4), gpu_ctx)
    w = q4.Q4Matrix.from_blocks(8, 64, synth.q4_blocks(1, 8, 64), gpu_ctx)
    with pytest.raises(q4.LghShapeError):
        q4.gemv_q4(w, np.zeros(32, dtype=np.float32), np.zeros(8, dtype=np.float32))
    with pytest.raises(q4.LghShapeError):
        q4.gemm_q4(w, np.zeros(64 * 3, dtype=np.float32), np.zeros(8 * 2, dtype=np.float32), 3)
    w2 = q4.Q4Matrix.from_blocks(16, 64, synth.q4_blocks(2, 16, 64), gpu_ctx)
    with pytest.raises(q4.LghShapeError):
        q4.gemv_q4_pair(w, w2, np.zeros(64, dtype=np.float32), np.zeros(8, dtype=np.float32),
                        np.zeros(16, dtype=np.float32))


def test_empty_is_noop(gpu_ctx):
    w = q4.Q4Matrix.from_blocks(0, 64, np.zeros(0, dtype=BLOCK_Q4), gpu_ctx)
    q4.gemv_q4(w, np.zeros(64, dtype=np.float32), np.zeros(0, dtype=np.float32))
    w2 = q4.Q4Matrix.from_blocks(8, 64, synth.q4_blocks(1, 8, 64), gpu_ctx)
    out = np.full((0, 8), 3.0, dtype=np.float32)
    q4.gemm_q4(w2, np.zeros((0, 64), dtype=np.float32), out, 0)


# ---- device pointers (torch tensors) ------------------------------------------------------------
def test_device_pointer_path_matches_host_path(gpu_ctx):
    import torch

    n, k, m = 4096, 2048, 24
    blocks = synth.q4_blocks(61, n, k)
    x = synth.activations(62, m, k)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    host1 = np.zeros(n, dtype=np.float32)
    q4.gemv_q4(w, np.ascontiguousarray(x[0]), host1)
    hostm = np.zeros((m, n), dtype=np.float32)
    q4.gemm_q4(w, x, hostm, m)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        xd = torch.from_numpy(x).cuda()
        y1 = torch.zeros(n, device="cuda")
        ym = torch.zeros(m, n, device="cuda")
        gpu_ctx.set_stream(stream.cuda_stream)
        try:
            q4.gemv_q4(w, xd[0], y1)
            q4.gemm_q4(w, xd, ym, m)
            stream.synchronize()
        finally:
            gpu_ctx.set_stream(None)
    assert np.array_equal(y1.cpu().numpy(), host1)
    assert np.array_equal(ym.cpu().numpy(), hostm)
    # device-resident raw blocks upload
    bd = torch.from_numpy(blocks.view(np.uint8).copy()).cuda()
    wd = q4.Q4Matrix.from_blocks(n, k, bd, gpu_ctx)
    assert wd.blocks().tobytes() == blocks.tobytes()


# ---- HIP graph replay and split-K determinism -------------------------------------------------
def test_split_k_gemv_is_deterministic(gpu_ctx, oracle):
    n, k = 1536, 10752  # several K slices
    blocks = synth.q4_blocks(81, n, k)
    x = synth.normal_f32(82, k)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    outs = []
    for _ in range(3):
        y = np.zeros(n, dtype=np.float32)
        q4.gemv_q4(w, x, y)
        outs.append(y)
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    assert_close(outs[0], oracle.gemv_q4(oracle.Q4Matrix(n, k, blocks), x, threads=8), what="split-K")


@pytest.mark.parametrize("mode", [_ffi.LGH_ASSIGN, _ffi.LGH_ADD_F64, _ffi.LGH_ADD_F32])
def test_split_k_reduce_vector_and_scalar_forms(gpu_ctx, oracle, mode):
    """The split-K reduce adds four outputs per thread when every m * n is a multiple of 4 and y
    is 16-byte aligned, else one: N=1536 (vector), N=1531 (odd: scalar) and N=1536 into a y one
    float past an aligned address (scalar), against the oracle and bit-equal between the forms."""
    import torch

    m, k = 65, 8192  # 65 tokens x 8192: three 32-token tiles, K split
    results = {}
    for n in (1536, 1531):
        blocks = synth.q4_blocks(70 + n, n, k)
        w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
        x = synth.activations(71, m, k)
        y0 = synth.activations(72 + n, m, n)
        xd = torch.from_numpy(x).cuda()
        buf = torch.zeros(m * n + 4, device="cuda")
        for off in (0, 1) if n == 1536 else (0,):
            y = buf[off:off + m * n].view(m, n)
            y.copy_(torch.from_numpy(y0))
            {_ffi.LGH_ASSIGN: q4.gemm_q4, _ffi.LGH_ADD_F64: q4.gemm_q4_add,
             _ffi.LGH_ADD_F32: q4.apply_add_inplace}[mode](w, xd, y, m)
            torch.cuda.synchronize()
            results[(n, off)] = y.cpu().numpy()
        ref = oracle.gemm_q4(oracle.Q4Matrix(n, k, blocks), x, m, threads=8)
        if mode == _ffi.LGH_ASSIGN:
            assert_close(results[(n, 0)], ref, what=f"n={n}")
        else:
            got = results[(n, 0)].astype(np.float64) - y0.astype(np.float64)
            assert_close(got, ref, atol=2e-4, what=f"n={n} mode={mode}")
        w.free()
    assert np.array_equal(results[(1536, 0)], results[(1536, 1)])


def test_graph_replay_matches_eager(gpu_ctx):
    """Capture GEMV (one slice and split-K), pair, AddF64 and GEMM into one
    graph; replay it several times with eager work in between and check every
    replay bit-exactly against the eager results."""
    import torch

    shapes = {"up": (8192, 1536), "down": (1536, 8192)}
    mats = {k: q4.Q4Matrix.from_blocks(n, kk, synth.q4_blocks(90 + i, n, kk), gpu_ctx)
            for i, (k, (n, kk)) in enumerate(shapes.items())}
    gate = q4.Q4Matrix.from_blocks(8192, 1536, synth.q4_blocks(95, 8192, 1536), gpu_ctx)
    stream = torch.cuda.Stream()
    gpu_ctx.set_stream(stream.cuda_stream)
    try:
        with torch.cuda.stream(stream):
            x1 = torch.from_numpy(synth.normal_f32(96, 1536)).cuda()
            x2 = torch.from_numpy(synth.normal_f32(97, 8192)).cuda()
            xm = torch.from_numpy(synth.activations(98, 64, 1536)).cuda()
            y0 = torch.from_numpy(synth.normal_f32(99, 1536)).cuda()
            outs = {"up": torch.empty(8192, device="cuda"), "g": torch.empty(8192, device="cuda"),
                    "u": torch.empty(8192, device="cuda"), "down": torch.empty(1536, device="cuda"),
                    "gemm": torch.empty(64, 8192, device="cuda")}

            def run():
                q4.gemv_q4(mats["up"], x1, outs["up"])
                q4.gemv_q4_pair(gate, mats["up"], x1, outs["g"], outs["u"])
                outs["down"].copy_(y0)
                q4.gemv_q4_add(mats["down"], x2, outs["down"])
                q4.gemm_q4(mats["up"], xm, outs["gemm"], 64)

            run()
            stream.synchronize()
            eager = {k: v.clone() for k, v in outs.items()}
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                run()
            for rep in range(3):
                for v in outs.values():
                    v.fill_(float("nan"))
                scratch = torch.empty(1536, device="cuda")
                q4.gemv_q4(mats["down"], x2, scratch)  # eager work between replays
                graph.replay()
                stream.synchronize()
                for k, v in outs.items():
                    assert torch.equal(v, eager[k]), f"replay {rep}: {k} differs"
            del graph
    finally:
        gpu_ctx.set_stream(None)
