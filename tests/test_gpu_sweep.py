"""Seeded random sweep of lgh_q4_gemm over its route boundaries (M = 1 | 2-4 | 5-64 | 65+, one or
several K slices, N not a multiple of any tile), all three accumulation modes and both act-quant
modes, against the oracle's scalar-order GEMM (gemv_q4.rs:499-544, 822-952).  The cases are drawn
once from a fixed seed, so every run checks the same shapes.
"""

import numpy as np
import pytest

from llmhost_amd import q4, synth
from llmhost_amd._ffi import LGH_ADD_F32, LGH_ADD_F64, LGH_ASSIGN

from .conftest import assert_close

pytestmark = pytest.mark.gpu

M_CHOICES = [1, 2, 3, 4, 5, 6, 15, 16, 17, 31, 32, 33, 63, 64, 65, 66, 100, 257]


def _cases(count=48, seed=20261202, budget=1.2e8):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        m = int(rng.choice(M_CHOICES))
        n = int(rng.integers(1, 3000))
        k = 32 * int(rng.integers(1, 220))
        if m * n * k > budget:
            continue
        out.append((m, n, k, int(rng.integers(0, 3)), bool(rng.integers(0, 2)), int(rng.integers(0, 1 << 30))))
    return out


CASES = _cases()


@pytest.mark.parametrize("m,n,k,mode,per_row,seed", CASES)
def test_gemm_sweep(gpu_ctx, oracle, m, n, k, mode, per_row, seed):
    blocks = synth.q4_blocks(seed, n, k)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    x = synth.activations(seed + 1, m, k)
    y0 = synth.normal_f32(seed + 2, m * n).reshape(m, n)
    got = y0.copy()
    gpu_ctx.set_act_quant(q4.ActQuant.PerRow if per_row else q4.ActQuant.PerBlock)
    try:
        q4._gemm(w, x, got, m, [LGH_ASSIGN, LGH_ADD_F64, LGH_ADD_F32][mode])
    finally:
        gpu_ctx.set_act_quant(q4.ActQuant.PerBlock)
    cw = oracle.Q4Matrix(n, k, blocks)
    prod = oracle.gemm_q4(cw, x, m, per_row=per_row, kernel=oracle.KERNEL_SCALAR, threads=8)
    if mode == 0:
        ref = prod
    elif mode == 1:
        ref = (y0.astype(np.float64) + prod.astype(np.float64)).astype(np.float32)
    else:
        ref = y0 + prod
    assert_close(got, ref, what=f"m={m} n={n} k={k} mode={mode} per_row={per_row}")


# Without split K, launches of >= 640 workgroups of 128 rows x 64 tokens (summed over the matrices
# of one call) take those tiles (each wave 32 rows x 64 tokens); smaller launches keep 128 x 32.
# Short K keeps the oracle fast; ragged M (a 64-token tile with a missing half), N and an odd
# block count cover the tile and pair tails.
WIDE = [(2048, 10752, 64), (2100, 3000, 96), (512, 10752, 96), (770, 10700, 64)]
NARROW = [(4096, 700, 128), (512, 8192, 96), (300, 10752, 64)]


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("m,n,k", WIDE)
def test_gemm_wide_tile_route(gpu_ctx, oracle, m, n, k, mode, per_row):
    test_gemm_sweep(gpu_ctx, oracle, m, n, k, mode, per_row, 37 * m + n + k + mode)


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("m,n,k", NARROW)
def test_gemm_below_wide_threshold(gpu_ctx, oracle, m, n, k, mode, per_row):
    test_gemm_sweep(gpu_ctx, oracle, m, n, k, mode, per_row, 31 * m + n + k + mode)


# Launches of fewer than 512 tiles of 128 x 32 that are not split run K groups inside the
# workgroup (four below 256 tiles with >= 4 block pairs, else two), and two K groups take the
# place of a two-way split on rows of 64..128 block pairs.  Pair counts that do not divide by the
# group count give groups of unequal length, the last ones partly or wholly without pairs.
K_GROUPS = [(512, 2048, 1536),  # 256 tiles, 24 pairs: two groups of 12
            (256, 4096, 4096),  # 256 tiles, 64 pairs: two groups in place of two splits
            (300, 4096, 4096),  # 320 tiles, 64 pairs: the same with a ragged last token tile
            (130, 1000, 2080),  # 40 tiles, 33 pairs: four groups of 9, 9, 9 and 6 pairs
            (100, 3000, 224),   # 96 tiles, 4 pairs: four groups of one pair
            (65, 256, 96),      # 6 tiles, 2 pairs: two groups of one pair
            (97, 200, 288)]     # 8 tiles, 5 pairs: four groups of 2, 2, 1 and 0 pairs


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("m,n,k", K_GROUPS)
def test_gemm_k_groups(gpu_ctx, oracle, m, n, k, mode, per_row):
    test_gemm_sweep(gpu_ctx, oracle, m, n, k, mode, per_row, 13 * m + n + k + mode)


@pytest.mark.parametrize("tokens", [2000, 256])  # 128 x 64 tiles (84 N groups x 32); 128 x 32 (84 x 8)
def test_gemm_large_routes_three_matrices(gpu_ctx, oracle, tokens):
    k, rows = 64, (4096, 4096, 2560)
    bl = [synth.q4_blocks(60 + j, n, k) for j, n in enumerate(rows)]
    gw = [q4.Q4Matrix.from_blocks(n, k, b, gpu_ctx) for n, b in zip(rows, bl)]
    x = synth.activations(64, tokens, k)
    outs = [np.full(tokens * n, np.nan, dtype=np.float32) for n in rows]
    q4.norm_gemv(gw, None, 1e-5, x, outs, tokens)
    for j, (o, n, b) in enumerate(zip(outs, rows, bl)):
        ref = oracle.gemm_q4(oracle.Q4Matrix(n, k, b), x, tokens, kernel=oracle.KERNEL_SCALAR, threads=8)
        assert_close(o, ref.ravel(), what=f"matrix {j}")


# M = 2..4 with rows of 65..256 blocks (K = 2080..8192): x is quantized once by the ActQ8 kernel
# and the batched GEMV reads the codes (ragged N, odd block counts).
BATCH_LONG = [(2, 1536, 8192), (3, 1000, 4096), (4, 2048, 8192), (4, 33, 6144), (2, 130, 4128),
              (3, 700, 3072), (4, 96, 2080)]


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("m,n,k", BATCH_LONG)
def test_batch_long_rows(gpu_ctx, oracle, m, n, k, mode, per_row):
    test_gemm_sweep(gpu_ctx, oracle, m, n, k, mode, per_row, 7 * m + n + k + mode)


# M = 49..64 over long rows (K >= 8192, or K >= 4096 with N >= 16384) takes the fp6 GEMM instead
# of the four-token-tile MMA kernel; M = 48 and K = 4096 with N = 4096 stay on the MMA kernel.
LONG_ROWS = [(64, 1536, 8192), (49, 300, 8224), (56, 16384, 4096), (48, 1536, 8192), (64, 4096, 4096)]


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("m,n,k", LONG_ROWS)
def test_long_rows_route(gpu_ctx, oracle, m, n, k, mode, per_row):
    test_gemm_sweep(gpu_ctx, oracle, m, n, k, mode, per_row, 11 * m + n + k + mode)


# M = 1 over rows of 65..128 blocks at N*matrices >= 16384: the GEMV takes 4 blocks per lane and
# 2 K slices (32 rows per workgroup); also for the gate/up pair.
@pytest.mark.parametrize("n,k", [(16384, 4096), (20000, 3072), (16400, 2080)])
def test_gemv_long_rows_wide(gpu_ctx, oracle, n, k):
    test_gemm_sweep(gpu_ctx, oracle, 1, n, k, 0, False, n + k)


def test_gemv_pair_long_rows(gpu_ctx, oracle):
    n, k = 8192, 4096
    bg, bu = synth.q4_blocks(71, n, k), synth.q4_blocks(72, n, k)
    wg = q4.Q4Matrix.from_blocks(n, k, bg, gpu_ctx)
    wu = q4.Q4Matrix.from_blocks(n, k, bu, gpu_ctx)
    x = synth.normal_f32(73, k)
    og, ou = np.zeros(n, np.float32), np.zeros(n, np.float32)
    q4.gemv_q4_pair(wg, wu, x, og, ou)
    assert_close(og, oracle.gemv_q4(oracle.Q4Matrix(n, k, bg), x, kernel=oracle.KERNEL_SCALAR, threads=8), what="gate")
    assert_close(ou, oracle.gemv_q4(oracle.Q4Matrix(n, k, bu), x, kernel=oracle.KERNEL_SCALAR, threads=8), what="up")
