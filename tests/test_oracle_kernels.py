"""Pins of the oracle's llm-cpu restatement (crates/llm-cpu/src/gemv_q4.rs,
pool.rs, crates/llm-engine/src/weights.rs:194-227).

Re-creates the reference's gemv_q4 tests (gemv_q4.rs:1080-1249) with their
formula-generated inputs, then pins the arithmetic against closed forms
computed with numpy primitives (float32 IEEE ops for the quantizer, exact
int64 dots and float64 sums for the matmuls).
"""

import numpy as np
import pytest

from llmhost_amd import synth
from llmhost_amd.formats import q4_nibbles

from .conftest import assert_close


# ---- ActQ8 (gemv_q4.rs:62-95) ------------------------------------------------------
def _round_away(y32: np.ndarray) -> np.ndarray:
    y = y32.astype(np.float64)
    return np.sign(y) * np.floor(np.abs(y) + 0.5)


def _actq_closed_form(x: np.ndarray, per_row: bool):
    x = x.astype(np.float32)
    k = x.size
    blocks = x.reshape(k // 32, 32)
    if per_row:
        scales = np.full(k // 32, np.float32(np.abs(x).max()) / np.float32(127.0), dtype=np.float32)
    else:
        scales = (np.abs(blocks).max(axis=1).astype(np.float32) / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(scales == 0, np.float32(0), np.float32(1.0) / scales).astype(np.float32)
    q = np.clip(_round_away((blocks * inv[:, None]).astype(np.float32)), -127, 127).astype(np.int8)
    return q.reshape(k), scales, q.astype(np.int32).sum(axis=1)


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("k", [32, 96, 1536])
def test_actq_matches_ieee_closed_form(oracle, per_row, k):
    x = synth.normal_f32(11 + k, k) * np.float32(3.0)
    x[5] = 0.0
    if k > 64:
        x[32:64] = 0.0  # an all-zero block: scale 0, codes 0 (per-block)
    qs, sc, su = oracle.act_quantize(x, per_row)
    q_ref, sc_ref, su_ref = _actq_closed_form(x, per_row)
    assert np.array_equal(sc.view(np.uint32), sc_ref.view(np.uint32))
    assert np.array_equal(qs, q_ref)
    assert np.array_equal(su, su_ref)


def test_actq_invariants(oracle):
    x = synth.activations(5, 7, 256)
    qs, sc, su = oracle.act_quantize(x, False)
    blocks = qs.reshape(7, 8, 32).astype(np.int32)
    assert np.all(np.abs(blocks).max(axis=2) == 127)  # amax element maps to +-127
    assert np.array_equal(blocks.sum(axis=2), su)
    err = np.abs(blocks * sc[..., None] - x.reshape(7, 8, 32))
    assert np.all(err <= sc[..., None] * 0.5000001 + 1e-12)


def test_actq_ties_and_zero(oracle):
    # amax = 127 -> scale = 1.0 exactly and inv = 1.0: codes are round(v).
    x = np.zeros(64, dtype=np.float32)
    x[:8] = [127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -1.5, 3.5]
    qs, sc, su = oracle.act_quantize(x, False)
    assert sc[0] == 1.0 and sc[1] == 0.0
    assert list(qs[:8]) == [127, 3, -3, 1, -1, 127, -2, 4]
    assert np.all(qs[32:] == 0) and su[1] == 0


def test_actq_per_row_uses_one_scale(oracle):
    x = synth.normal_f32(2, 512)
    _, sc, _ = oracle.act_quantize(x, True)
    assert np.all(sc == np.float32(np.abs(x).max()) / np.float32(127))


# ---- integer block dots (gemv_q4.rs:959-966, 1080-1102) ---------------------------------
def _pattern_block(seed):
    i = np.arange(32)
    w = (((i * 17 + seed) % 21) - 10).astype(np.float32) * np.float32(0.25)
    a = (((i * 9 + seed) % 25) - 12).astype(np.int8)
    return w, a


def test_vnni_identity_matches_scalar_dot(oracle):
    """vnni_and_avx2_match_scalar_dot (gemv_q4.rs:1090-1102)."""
    for seed in range(16):
        w, a = _pattern_block(seed)
        blk = oracle.quantize_q4(w)
        scalar = oracle.dot_q4_q8(blk, a)
        assert oracle.dot_q4_q8_offset(blk, a, int(a.astype(np.int32).sum())) == scalar
        # textbook integer dot of the decoded nibbles
        assert scalar == int(np.dot(q4_nibbles(blk)[0].astype(np.int64), a.astype(np.int64)))


def test_block_dots_random_exhaustive_extremes(oracle):
    rng = np.random.default_rng(9)
    blocks = synth.q4_blocks(4, 64, 32)
    for b in range(64):
        a = rng.integers(-127, 128, 32, dtype=np.int8)
        if b == 0:
            a[:] = -127
            blocks["qs"][b] = 0x88  # all nibbles -8: extreme positive dot
        ref = int(np.dot(q4_nibbles(blocks[b]).astype(np.int64), a.astype(np.int64)))
        assert oracle.dot_q4_q8(blocks[b], a) == ref
    q8 = synth.q8_blocks(5, 16, 32)
    for b in range(16):
        a = rng.integers(-127, 128, 32, dtype=np.int8)
        assert oracle.dot_q8_q8(q8[b], a) == int(np.dot(q8["qs"][b].astype(np.int64), a.astype(np.int64)))


# ---- GEMV (gemv_q4.rs:1104-1249) ------------------------------------------------------------
def _formula(n, k, wmul, wmod, woff, wscale, xmul, xmod, xoff, xscale):
    w = ((((np.arange(n * k) * wmul) % wmod) - woff).astype(np.float32) * np.float32(wscale)).astype(np.float32)
    x = ((((np.arange(k) * xmul) % xmod) - xoff).astype(np.float32) * np.float32(xscale)).astype(np.float32)
    return w, x


def _gemv_f64(blocks, n, k, qs, scales):
    """Closed form: sum_kb idot * sw * sa in float64 (idot exact int64)."""
    nib = q4_nibbles(blocks).reshape(n, k // 32, 32).astype(np.int64)
    idot = np.einsum("nbi,bi->nb", nib, qs.reshape(k // 32, 32).astype(np.int64))
    sw = blocks["scale"].view(np.float16).astype(np.float64).reshape(n, k // 32)
    return (idot * sw * scales.astype(np.float64)[None, :]).sum(axis=1)


def test_gemv_kernels_agree(oracle):
    """gemv_kernels_agree (gemv_q4.rs:1104-1140): n=17 (ragged tile), k=64."""
    n, k = 17, 64
    w, x = _formula(n, k, 13, 19, 9, 0.15, 7, 15, 7, 0.2)
    mat = oracle.Q4Matrix.from_f32(w, n, k)
    qs, sc, _ = oracle.act_quantize(x)
    outs = {kern: oracle.gemv_q4_prep(mat, qs, sc, kernel=kern)
            for kern in (oracle.KERNEL_SCALAR, oracle.KERNEL_AVX2, oracle.KERNEL_VNNI)}
    s = outs[oracle.KERNEL_SCALAR]
    for kern, o in outs.items():
        assert np.all(np.abs(o - s) <= 1e-6 * (1 + np.abs(s))), kern
    # scalar and AVX2 share the fold order exactly
    assert np.array_equal(outs[oracle.KERNEL_AVX2], s)


def test_packed_gemv_matches_block_dots_and_closed_form(oracle):
    """packed_gemv_matches_block_dots (gemv_q4.rs:1197-1249)."""
    n, k = 17, 64
    w, x = _formula(n, k, 13, 19, 9, 0.15, 7, 15, 7, 0.2)
    blocks = oracle.quantize_q4(w)
    qs, sc, _ = oracle.act_quantize(x)
    sw = blocks["scale"].view(np.float16).astype(np.float32)
    expected = np.zeros(n, dtype=np.float32)
    for row in range(n):
        acc = np.float32(0)
        for b in range(k // 32):
            idot = oracle.dot_q4_q8(blocks[row * 2 + b], qs[b * 32:(b + 1) * 32])
            acc = np.float32(acc + np.float32(np.float32(idot) * sw[row * 2 + b] * sc[b]))
        expected[row] = acc
    mat = oracle.Q4Matrix(n, k, blocks)
    for kern in (oracle.KERNEL_SCALAR, oracle.KERNEL_VNNI):
        got = oracle.gemv_q4_prep(mat, qs, sc, kernel=kern)
        assert np.all(np.abs(got - expected) <= 1e-6 * (1 + np.abs(expected)))
    assert_close(oracle.gemv_q4(mat, x), _gemv_f64(blocks, n, k, qs, sc), atol=1e-6, rtol=1e-6,
                 what="closed form")


def test_gemv_pool_matches_serial(oracle):
    """gemv_pool_matches_serial (gemv_q4.rs:1142-1165)."""
    n, k = 128, 64
    w, x = _formula(n, k, 3, 17, 8, 0.1, 5, 11, 5, 0.2)
    mat = oracle.Q4Matrix.from_f32(w, n, k)
    serial = oracle.gemv_q4(mat, x, threads=1)
    pooled = oracle.gemv_q4(mat, x, threads=4)
    assert np.all(np.abs(serial - pooled) <= 1e-6 * (1 + np.abs(serial)))


@pytest.mark.parametrize("n,k", [(1536, 1536), (300, 2048), (64, 8192)])
def test_gemv_seeded_closed_form(oracle, n, k):
    blocks = synth.q4_blocks(100 + n, n, k)
    x = synth.normal_f32(200 + k, k)
    mat = oracle.Q4Matrix(n, k, blocks)
    qs, sc, _ = oracle.act_quantize(x)
    ref = _gemv_f64(blocks, n, k, qs, sc)
    for kern in (oracle.KERNEL_SCALAR, oracle.KERNEL_VNNI):
        assert_close(oracle.gemv_q4(mat, x, kernel=kern, threads=4), ref, what=f"kernel {kern}")


def test_gemv_add_f64_closed_form(oracle):
    n, k = 100, 256
    blocks = synth.q4_blocks(1, n, k)
    x = synth.normal_f32(2, k)
    y0 = synth.normal_f32(3, n) * np.float32(1e4)
    mat = oracle.Q4Matrix(n, k, blocks)
    g = oracle.gemv_q4(mat, x)
    got = oracle.gemv_q4(mat, x, out=y0.copy(), add=True)
    ref = (y0.astype(np.float64) + g.astype(np.float64)).astype(np.float32)
    assert np.array_equal(got, ref)


def test_gemv_per_row(oracle):
    n, k = 50, 512
    blocks = synth.q4_blocks(8, n, k)
    x = synth.normal_f32(9, k)
    mat = oracle.Q4Matrix(n, k, blocks)
    qs, sc, _ = oracle.act_quantize(x, per_row=True)
    assert_close(oracle.gemv_q4(mat, x, per_row=True), _gemv_f64(blocks, n, k, qs, sc), what="per row")


def test_pair_equals_two_gemvs(oracle):
    n, k = 96, 320
    bg, bu = synth.q4_blocks(1, n, k), synth.q4_blocks(2, n, k)
    x = synth.normal_f32(3, k)
    mg, mu = oracle.Q4Matrix(n, k, bg), oracle.Q4Matrix(n, k, bu)
    og, ou = oracle.gemv_q4_pair(mg, mu, x, threads=3)
    assert np.array_equal(og, oracle.gemv_q4(mg, x))
    assert np.array_equal(ou, oracle.gemv_q4(mu, x))


# ---- GEMM (gemv_q4.rs:1167-1195) ------------------------------------------------------------
def test_gemm_matches_per_token_gemv(oracle):
    """gemm_matches_per_token_gemv: n=48, k=64, m=20."""
    n, k, m = 48, 64, 20
    w = ((((np.arange(n * k) * 3) % 17) - 8).astype(np.float32) * np.float32(0.1)).astype(np.float32)
    x = ((((np.arange(m * k) * 5) % 11) - 5).astype(np.float32) * np.float32(0.2)).astype(np.float32)
    mat = oracle.Q4Matrix.from_f32(w, n, k)
    gemm = oracle.gemm_q4(mat, x, m, threads=4)
    gemv = np.stack([oracle.gemv_q4(mat, x[t * k:(t + 1) * k]) for t in range(m)])
    assert np.all(np.abs(gemm - gemv) <= 1e-5 * (1 + np.abs(gemv)))


@pytest.mark.parametrize("per_row", [False, True])
def test_gemm_closed_form_and_add(oracle, per_row):
    n, k, m = 70, 192, 9
    blocks = synth.q4_blocks(21, n, k)
    x = synth.activations(22, m, k)
    mat = oracle.Q4Matrix(n, k, blocks)
    qs, sc, _ = oracle.act_quantize(x, per_row)
    ref = np.stack([_gemv_f64(blocks, n, k, qs[t], sc[t]) for t in range(m)])
    for kern in (oracle.KERNEL_SCALAR, oracle.KERNEL_VNNI):
        got = oracle.gemm_q4(mat, x, m, per_row=per_row, kernel=kern, threads=2)
        assert_close(got, ref, what=f"gemm kernel {kern}")
    y0 = synth.activations(23, m, n)
    g = oracle.gemm_q4(mat, x, m, per_row=per_row)
    got = oracle.gemm_q4(mat, x, m, out=y0.copy(), add=True, per_row=per_row)
    assert np.array_equal(got, (y0.astype(np.float64) + g.astype(np.float64)).astype(np.float32))


# ---- AMX-INT8 tiles (crates/llm-cpu/src/amx.rs) --------------------------------------------------
@pytest.fixture
def amx_host(oracle):
    if not oracle.amx_ready():
        pytest.skip("the host cannot run AMX-INT8 tiles (no AMX-INT8 in CPUID, or the kernel "
                    "refused the tile-data permission)")


@pytest.mark.usefixtures("amx_host")
def test_amx_gemm_matches_gemv(oracle):
    """amx_gemm_matches_gemv_when_available (amx.rs:526-557): n=48, k=64, m=40, two threads."""
    n, k, m = 48, 64, 40
    w = ((((np.arange(n * k) * 3) % 17) - 8).astype(np.float32) * np.float32(0.1)).astype(np.float32)
    x = ((((np.arange(m * k) * 5) % 11) - 5).astype(np.float32) * np.float32(0.2)).astype(np.float32)
    mat = oracle.Q4Matrix.from_f32(w, n, k)
    gemm = oracle.gemm_q4(mat, x, m, kernel=oracle.KERNEL_AMX, threads=2)
    gemv = np.stack([oracle.gemv_q4(mat, x[t * k:(t + 1) * k]) for t in range(m)])
    assert np.all(np.abs(gemm - gemv) <= 1e-4 * (1 + np.abs(gemv)))


@pytest.mark.usefixtures("amx_host")
@pytest.mark.parametrize("threads", [1, 4])
@pytest.mark.parametrize("m,n,k", [(16, 64, 64), (17, 96, 96), (40, 48, 2048), (100, 160, 288), (33, 32, 1536)])
def test_amx_equals_vnni_on_whole_tiles(oracle, m, n, k, threads):
    """On 16-column tiles the AMX fold is fma(f32(c), sw * sa, acc) per block in ascending order,
    the VNNI kernel's own operation (fold_c_avx512, amx.rs:293-320; gemv_q4.rs:930-936): the two
    agree bit for bit, and match the exact float64 reference within the output tolerance."""
    if not oracle.cpu_has("avx512vnni"):
        pytest.skip("no VNNI-512 kernel to compare with")
    blocks = synth.q4_blocks(700 + m + n + k, n, k)
    x = synth.activations(701 + m, m, k)
    mat = oracle.Q4Matrix(n, k, blocks)
    amx = oracle.gemm_q4(mat, x, m, kernel=oracle.KERNEL_AMX, threads=threads)
    vnni = oracle.gemm_q4(mat, x, m, kernel=oracle.KERNEL_VNNI, threads=threads)
    assert np.array_equal(amx.view(np.uint32), vnni.view(np.uint32))
    qs, sc, _ = oracle.act_quantize(x, False)
    ref = np.stack([_gemv_f64(blocks, n, k, qs[t], sc[t]) for t in range(m)])
    assert_close(amx, ref, what="amx vs exact")


@pytest.mark.usefixtures("amx_host")
@pytest.mark.parametrize("m,n,k", [(16, 17, 64), (50, 1000, 128), (31, 70, 192)])
def test_amx_partial_tiles_within_tolerance(oracle, m, n, k):
    """A partial last tile (n % 16 != 0) folds as acc + (c * sw) * sa (fold_c, amx.rs:280-288):
    within the output tolerance of the exact reference, and equal to VNNI on the whole tiles."""
    blocks = synth.q4_blocks(710 + m + n, n, k)
    x = synth.activations(711 + m, m, k)
    mat = oracle.Q4Matrix(n, k, blocks)
    amx = oracle.gemm_q4(mat, x, m, kernel=oracle.KERNEL_AMX, threads=2)
    qs, sc, _ = oracle.act_quantize(x, False)
    ref = np.stack([_gemv_f64(blocks, n, k, qs[t], sc[t]) for t in range(m)])
    assert_close(amx, ref, what="amx partial tiles")
    whole = n // 16 * 16
    if whole and oracle.cpu_has("avx512vnni"):
        vnni = oracle.gemm_q4(mat, x, m, kernel=oracle.KERNEL_VNNI, threads=2)
        assert np.array_equal(amx[:, :whole].view(np.uint32), vnni[:, :whole].view(np.uint32))


@pytest.mark.usefixtures("amx_host")
def test_amx_dispatch_follows_gemm_q4_mode(oracle):
    """gemv_q4.rs:711: the detected kernel takes AMX for m >= 16 without add; m = 15, and
    gemm_q4_add at any m, stay on the tile kernels."""
    n, k = 40, 96  # a partial last tile, where AMX and VNNI round differently
    blocks = synth.q4_blocks(720, n, k)
    mat = oracle.Q4Matrix(n, k, blocks)
    for m, want in ((16, oracle.KERNEL_AMX), (15, oracle.KERNEL_VNNI)):
        x = synth.activations(721 + m, m, k)
        auto = oracle.gemm_q4(mat, x, m, kernel=oracle.KERNEL_DETECT)
        forced = oracle.gemm_q4(mat, x, m, kernel=want)
        assert np.array_equal(auto.view(np.uint32), forced.view(np.uint32)), m
    x = synth.activations(730, 20, k)
    y0 = synth.activations(731, 20, n)
    add = oracle.gemm_q4(mat, x, 20, out=y0.copy(), add=True)
    tile = oracle.gemm_q4(mat, x, 20, kernel=oracle.KERNEL_VNNI)
    assert np.array_equal(add, (y0.astype(np.float64) + tile.astype(np.float64)).astype(np.float32))


# ---- Q8_0 GEMV (weights.rs:194-227) ------------------------------------------------------------
def test_q8_apply_closed_form(oracle):
    n, k, tokens = 77, 256, 3
    blocks = synth.q8_blocks(31, n, k)
    x = synth.activations(32, tokens, k)
    got = oracle.q8_apply(blocks, n, k, x, tokens, threads=2)
    qs, sc, _ = oracle.act_quantize(x, False)
    wq = blocks["qs"].reshape(n, k // 32, 32).astype(np.int64)
    sw = blocks["scale"].view(np.float16).astype(np.float64).reshape(n, k // 32)
    for t in range(tokens):
        idot = np.einsum("nbi,bi->nb", wq, qs[t].reshape(k // 32, 32).astype(np.int64))
        ref = (idot * sw * sc[t].astype(np.float64)[None, :]).sum(axis=1)
        assert_close(got[t], ref, what=f"token {t}")


# ---- pool (pool.rs:212-221, 356-426) -------------------------------------------------------------
@pytest.mark.parametrize("nthreads", [1, 3, 4, 7, 64])
@pytest.mark.parametrize("n", [0, 1, 5, 64, 1000])
def test_thread_ranges_cover_without_overlap(oracle, nthreads, n):
    covered = []
    for tid in range(nthreads):
        s, e = oracle.thread_range(tid, nthreads, n)
        assert s <= e
        covered.extend(range(s, e))
    assert covered == list(range(n))
