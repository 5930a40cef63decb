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
