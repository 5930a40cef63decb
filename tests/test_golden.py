"""Committed known-answer vectors (tests/golden/fixtures.npz, written by
tests/golden/make_golden.py from numpy restatements of the reference's
arithmetic) against the oracle (CPU) and against the GPU library.

Integer outputs (activation codes / sums, weight codes, block dots) and the
scale bit patterns must match exactly; fp32 matmul outputs match the
reference operation order exactly on the oracle's scalar kernel and within
|d| <= 1e-4 + 1e-5 |ref| on the GPU, whose summation order differs.
"""

import os

import numpy as np
import pytest

import oracle
from llmhost_amd import formats, q4

from .conftest import assert_close

FX = np.load(os.path.join(os.path.dirname(__file__), "golden", "fixtures.npz"))


def _blocks_q4(nib, bits):
    return formats.q4_from_nibbles(nib, bits)


# ---- the oracle reproduces every vector ---------------------------------------------------
@pytest.mark.parametrize("tag,per_row", [("block", False), ("row", True)])
def test_oracle_act_quant_fixture(tag, per_row):
    qs, sc, su = oracle.act_quantize(FX["act_x"], per_row)
    assert np.array_equal(qs, FX[f"act_qs_{tag}"])
    assert np.array_equal(sc.view(np.uint32), FX[f"act_sc_{tag}"].view(np.uint32))
    assert np.array_equal(su, FX[f"act_sum_{tag}"])


def test_fixture_act_quant_edge_cases_are_the_rust_semantics():
    """Spot values fixed by the reference's arithmetic, independent of any restatement."""
    qs, sc, su = FX["act_qs_block"], FX["act_sc_block"], FX["act_sum_block"]
    assert list(qs[0, 32:40]) == [127, 3, -3, 1, -1, 127, -2, 4]   # .5 ties away from zero
    assert sc[0, 0] == 0.0 and not qs[0, :32].any()                 # zero block
    # denormal block: 1 / scale overflows to inf, so every nonzero input saturates and
    # 0 * inf = NaN casts to 0 (Rust `as i8`)
    assert qs[3, 0] == 0 and (qs[3, 1:32] == 127).all() and su[3, 0] == 31 * 127
    assert not qs[3, 32:64].any() and sc[3, 1] == 0.0              # signed zeros
    assert set(np.abs(qs[3, 64:96]).tolist()) == {127}             # +-3e38


def test_oracle_weight_quantizers_fixture():
    b4 = oracle.quantize_q4(FX["qw_x"])
    assert b4.tobytes() == _blocks_q4(FX["q4_nib"], FX["q4_bits"]).tobytes()
    b8 = oracle.quantize_q8_0(FX["qw_x"])
    assert np.array_equal(b8["qs"], FX["q8_q"]) and np.array_equal(b8["scale"], FX["q8_bits"])


def test_oracle_block_dots_fixture():
    blocks = _blocks_q4(FX["dot_nib"], np.full(len(FX["dot_nib"]), 0x3C00, np.uint16))
    got = np.array([oracle.dot_q4_q8(blocks[i], FX["dot_act"][i]) for i in range(len(blocks))])
    assert np.array_equal(got, FX["dot_q4"])
    assert FX["dot_q4"][-3] == 32512 and FX["dot_q4"][-2] == 7 * 127 * 32


@pytest.mark.parametrize("tag,n,k", [("a", 17, 64), ("b", 128, 64)])
def test_oracle_gemv_fixture(tag, n, k):
    mat = oracle.Q4Matrix.from_f32(FX[f"gemv_{tag}_w"], n, k)
    for kernel in (oracle.KERNEL_SCALAR,):
        y = oracle.gemv_q4(mat, FX[f"gemv_{tag}_x"], kernel=kernel)
        assert np.array_equal(y.view(np.uint32), FX[f"gemv_{tag}_y"].view(np.uint32))
    y = oracle.gemv_q4(mat, FX[f"gemv_{tag}_x"], kernel=oracle.KERNEL_VNNI)
    assert_close(y, FX[f"gemv_{tag}_y"], what="vnni")
    ya = oracle.gemv_q4(mat, FX[f"gemv_{tag}_x"], out=FX[f"gemv_{tag}_y0"].copy(), add=True,
                        kernel=oracle.KERNEL_SCALAR)
    assert np.array_equal(ya.view(np.uint32), FX[f"gemv_{tag}_yadd"].view(np.uint32))


def test_oracle_gemm_and_q8_fixture():
    mat = oracle.Q4Matrix.from_f32(FX["gemm_w"], 48, 64)
    y = np.asarray(oracle.gemm_q4(mat, FX["gemm_x"], 20, kernel=oracle.KERNEL_SCALAR)).reshape(20, 48)
    assert np.array_equal(y.view(np.uint32), FX["gemm_y"].view(np.uint32))
    y = oracle.q8_apply(oracle.quantize_q8_0(FX["q8_w"]), 33, 96, FX["q8_x"])
    assert np.array_equal(np.asarray(y).view(np.uint32), FX["q8_y"].view(np.uint32))


# ---- the GPU library against the same vectors ------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("tag,per_row", [("block", False), ("row", True)])
def test_gpu_act_quant_fixture(gpu_ctx, tag, per_row):
    act = (q4.ActQ8.quantize_row if per_row else q4.ActQ8.quantize)(FX["act_x"], gpu_ctx)
    assert np.array_equal(act.qs, FX[f"act_qs_{tag}"])
    assert np.array_equal(act.scales.view(np.uint32), FX[f"act_sc_{tag}"].view(np.uint32))
    assert np.array_equal(act.sums, FX[f"act_sum_{tag}"])


@pytest.mark.gpu
def test_gpu_weight_quantizers_and_dots_fixture(gpu_ctx):
    x = FX["qw_x"].reshape(-1, 32)
    w4 = q4.Q4Matrix.from_f32(x, x.shape[0], 32, gpu_ctx)
    assert w4.blocks().tobytes() == _blocks_q4(FX["q4_nib"], FX["q4_bits"]).tobytes()
    w8 = q4.Q8Matrix.from_f32(x, x.shape[0], 32, gpu_ctx).blocks()
    assert np.array_equal(w8["qs"], FX["q8_q"]) and np.array_equal(w8["scale"], FX["q8_bits"])
    blocks = _blocks_q4(FX["dot_nib"], np.full(len(FX["dot_nib"]), 0x3C00, np.uint16))
    assert np.array_equal(q4.q4_block_dots(blocks, FX["dot_act"], gpu_ctx), FX["dot_q4"])
    # the same dots through the GEMM's matrix-core path: one row per block, one token each
    nb = len(blocks)
    wm = q4.Q4Matrix.from_blocks(nb, 32, blocks, gpu_ctx)
    got = q4.q4_mfma_block_dots(wm, FX["dot_act"], nb)      # [token][row][0]
    assert np.array_equal(np.diagonal(got[:, :, 0]), FX["dot_q4"])


@pytest.mark.gpu
@pytest.mark.parametrize("tag,n,k", [("a", 17, 64), ("b", 128, 64)])
def test_gpu_gemv_fixture(gpu_ctx, tag, n, k):
    w = q4.Q4Matrix.from_f32(FX[f"gemv_{tag}_w"], n, k, gpu_ctx)
    y = np.zeros(n, np.float32)
    q4.gemv_q4(w, FX[f"gemv_{tag}_x"], y)
    assert_close(y, FX[f"gemv_{tag}_y"], what="gemv")
    ya = FX[f"gemv_{tag}_y0"].copy()
    q4.gemv_q4_add(w, FX[f"gemv_{tag}_x"], ya)
    assert_close(ya, FX[f"gemv_{tag}_yadd"], what="gemv add")


@pytest.mark.gpu
def test_gpu_gemm_and_q8_fixture(gpu_ctx):
    w = q4.Q4Matrix.from_f32(FX["gemm_w"], 48, 64, gpu_ctx)
    y = np.zeros((20, 48), np.float32)
    q4.gemm_q4(w, FX["gemm_x"], y, 20)
    assert_close(y, FX["gemm_y"], what="gemm")
    w8 = q4.Q8Matrix.from_f32(FX["q8_w"], 33, 96, gpu_ctx)
    y = np.zeros(33, np.float32)
    q4.q8_apply(w8, FX["q8_x"], 1, y)
    assert_close(y, FX["q8_y"], what="q8")
