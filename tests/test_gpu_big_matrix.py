"""A Q4 matrix whose GEMM operand image would pass 2 GiB (31-bit buffer offsets) has none: the
calls that would take the GEMM -- m >= 65, m = 49..64 over long rows, m = 1 and the prepared
GEMV with k > 32768 -- run the matrix-core batch kernel on the nibble planes instead, 64 tokens
per launch (llm-cpu's gemm_q4 / gemv_q4 / gemv_q4_prep have no such limit, gemv_q4.rs:344-393,
686-722).  Rows are independent, so the device's output is checked on sampled rows: against the
exact value of the same ActQ8 codes (every term is exact in f64) within the output gate plus
the f32 summation allowance of 2048 blocks, as the oracle is."""

import ctypes as C

import numpy as np
import pytest

from llmhost_amd import _ffi, q4, synth
from llmhost_amd.formats import BLOCK_Q4

from .conftest import assert_close_with_flips, q4_exact_terms, summation_allowance

pytestmark = pytest.mark.gpu

N, K = 37216, 65536  # (1163 + 8) 32-row tiles x 1024 block pairs x 1792 B = 2,148,532,224 B > 2^31
ROWS = np.r_[0:48, N - 40:N]


@pytest.fixture(scope="module")
def big(gpu_ctx):
    print(f"[big] uploading {N} x {K}", flush=True)
    rng = np.random.default_rng(4242)
    nb = N * (K // 32)
    blocks = np.empty(nb, dtype=BLOCK_Q4)
    blocks["qs"] = rng.integers(0, 256, size=(nb, 16), dtype=np.uint8)
    blocks["scale"] = rng.uniform(1e-3, 2e-2, size=nb).astype(np.float16).view(np.uint16)
    w = q4.Q4Matrix.from_blocks(N, K, blocks, gpu_ctx)
    sub = np.ascontiguousarray(blocks.reshape(N, K // 32)[ROWS]).reshape(-1)
    del blocks
    yield w, sub
    w.free()
    gpu_ctx.trim()


def _check(oracle, sub, x, got, what, per_row=False):
    m = x.shape[0]
    qs, sa, _ = oracle.act_quantize(x, per_row)
    exact, R = q4_exact_terms(sub, len(ROWS), K, qs, sa)
    allow = summation_allowance(R, K // 32)
    mat = oracle.Q4Matrix(len(ROWS), K, sub)
    ref = oracle.gemm_q4(mat, x, m, per_row=per_row, threads=8) if m > 1 else \
        oracle.gemv_q4(mat, x[0], per_row=per_row, threads=8)[None]
    assert_close_with_flips(ref, exact, allow, what=f"oracle vs exact, {what}")
    assert_close_with_flips(got[:, ROWS], exact, allow, what=f"device vs exact, {what}")


def test_big_matrix_has_no_gemm_image(big):
    w, _ = big
    with pytest.raises(_ffi.LghShapeError):
        w.prepare_gemm()
    assert w.device_bytes() < N * (K // 32) * 18 + 4096  # the planes only


@pytest.mark.parametrize("m", [1, 64, 70])
def test_big_matrix_gemm_routes(gpu_ctx, oracle, big, m):
    """m = 1 (k > 32768), m = 64 (four token tiles over long rows) and m = 70 (two launches of
    64 + 6 tokens), Assign and AddF64."""
    w, sub = big
    print(f"[big] m={m}", flush=True)
    x = synth.activations(500 + m, m, K)
    got = np.zeros((m, N), np.float32)
    q4.gemm_q4(w, x, got, m) if m > 1 else q4.gemv_q4(w, x[0], got[0])
    _check(oracle, sub, x, got, f"m={m}")
    y0 = synth.activations(600 + m, m, N)
    added = y0.copy()
    q4.gemm_q4_add(w, x, added, m) if m > 1 else q4.gemv_q4_add(w, x[0], added[0])
    assert np.array_equal(added, (y0.astype(np.float64) + got.astype(np.float64)).astype(np.float32))


def test_big_matrix_per_row_and_prep(gpu_ctx, oracle, big):
    """PerRow act-quant over 70 tokens, and gemv_q4_prep (k > 32768) on ActQ8 codes: the codes are
    turned into the matrix-core image directly; the result equals the GEMV of the same x."""
    w, sub = big
    x = synth.activations(700, 70, K)
    gpu_ctx.set_act_quant(q4.ActQuant.PerRow)
    try:
        got = np.zeros((70, N), np.float32)
        q4.gemm_q4(w, x, got, 70)
    finally:
        gpu_ctx.set_act_quant(q4.ActQuant.PerBlock)
    _check(oracle, sub, x, got, "per row", per_row=True)
    acts = q4.ActQ8.quantize(x[3], gpu_ctx)
    prep = np.zeros(N, np.float32)
    q4.gemv_q4_prep(w, acts, prep)
    direct = np.zeros(N, np.float32)
    q4.gemv_q4(w, x[3], direct)
    assert np.array_equal(prep, direct)
    _check(oracle, sub, x[3:4], prep[None], "prep")


def test_big_matrix_noalloc(gpu_ctx, big):
    """The entry point that allocates nothing serves it too (no image to prepare): bit-equal to
    lgh_q4_gemm_dev, twice, the second call smaller."""
    import torch

    w, _ = big
    lib = _ffi.lib()
    for m in (70, 5):
        x = torch.from_numpy(synth.activations(800 + m, m, K)).cuda()
        want = torch.zeros(m, N, device="cuda")
        got = torch.full((m, N), 7.0, device="cuda")
        torch.cuda.synchronize()  # the library runs on its own stream
        for fn, y in ((lib.lgh_q4_gemm_dev, want), (lib.lgh_q4_gemm_dev_noalloc, got)):
            gpu_ctx.check(fn(gpu_ctx.handle, w.handle, C.c_void_p(x.data_ptr()), C.c_void_p(y.data_ptr()), m,
                             _ffi.LGH_ASSIGN))
        gpu_ctx.sync()
        assert torch.equal(got, want), m
