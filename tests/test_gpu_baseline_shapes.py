"""Parity at the exact shapes the benchmark times, against the oracle's production (VNNI-512)
kernel, plus the steady state of both GEMM tile forms' pipelines.

Shapes: the ragged batched GEMMs (M = 4 / 16 / 64, K = 2048, N = 8192), the four prefill GEMMs
(M = 512 / 2048 x K = 2048, N = 10752 and K = 10752, N = 2048), the decode GEMVs of the headline
step and of the 16-layer sweep, and the Q8_0 GEMV.  Inputs are the benchmark's generators.
"""

import numpy as np
import pytest

from llmhost_amd import q4, synth

from .conftest import assert_close

pytestmark = pytest.mark.gpu


def _gemm_vs_oracle(ctx, oracle, m, n, k, seed, scalar=False):
    print(f"[shape] m={m} n={n} k={k}", flush=True)
    blocks = synth.q4_blocks(seed, n, k)
    x = synth.activations(seed + 1, m, k)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, ctx)
    got = np.zeros((m, n), dtype=np.float32)
    q4.gemm_q4(w, x, got, m)
    mat = oracle.Q4Matrix(n, k, blocks)
    assert_close(got, oracle.gemm_q4(mat, x, m, kernel=oracle.KERNEL_VNNI, threads=8), what="vs vnni")
    if scalar:
        assert_close(got, oracle.gemm_q4(mat, x, m, kernel=oracle.KERNEL_SCALAR, threads=8), what="vs scalar")
    w.free()
    return got


@pytest.mark.parametrize("m", [4, 16, 64])
def test_ragged_gemm_benchmark_shape(gpu_ctx, oracle, m):
    """Ragged batches: M rows packed from sequences of 1-8 tokens (rows are independent, so the
    packing only sets M), K = 2048, N = 8192."""
    _gemm_vs_oracle(gpu_ctx, oracle, m, 8192, 2048, 300 + m, scalar=True)


@pytest.mark.parametrize("m,n,k", [(512, 10752, 2048), (512, 2048, 10752), (2048, 10752, 2048),
                                   (2048, 2048, 10752)])
def test_prefill_gemm_benchmark_shape(gpu_ctx, oracle, m, n, k):
    """K = 2048, N = 10752 (128 x 64 workgroup tiles: 672 / 2688 of them at M = 512 / 2048, 32
    block pairs); K = 10752, N = 2048 (128 x 32 tiles, 168 block pairs: split K at M = 512, 1024
    workgroups at M = 2048)."""
    _gemm_vs_oracle(gpu_ctx, oracle, m, n, k, 400 + m + k)


@pytest.mark.parametrize("k", [256, 288])
@pytest.mark.parametrize("m", [2000, 256])
def test_large_gemm_pipeline_steady_state(gpu_ctx, oracle, m, k):
    """Past the pipeline fill each stage buffer is refilled after it was computed: 4 and 5 block
    pairs (an even and an odd count) at N = 10752 run that steady state on the 128 x 64 tile form
    (M = 2000, a ragged last token tile) and on 128 x 32 tiles (M = 256: 336 workgroups of
    128 x 64 would be too few), against the oracle's scalar (reference-order) kernel."""
    _gemm_vs_oracle(gpu_ctx, oracle, m, 10752, k, 500 + k + m, scalar=True)


@pytest.mark.parametrize("n,k", [(1536, 1536), (8192, 1536), (1536, 8192), (2048, 1536)])
def test_decode_gemv_benchmark_shape(gpu_ctx, oracle, n, k):
    """The headline step's up / down GEMVs, the sweep's q/k/v (2048 x 1536) and o (1536 x 1536)."""
    blocks = synth.q4_blocks(600 + n + k, n, k)
    x = synth.normal_f32(601 + k, k)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    got = np.zeros(n, dtype=np.float32)
    q4.gemv_q4(w, x, got)
    mat = oracle.Q4Matrix(n, k, blocks)
    assert_close(got, oracle.gemv_q4(mat, x, kernel=oracle.KERNEL_SCALAR, threads=8), what="vs scalar")
    assert_close(got, oracle.gemv_q4(mat, x, kernel=oracle.KERNEL_VNNI, threads=8), what="vs vnni")
    w.free()


def test_q8_gemv_benchmark_shape(gpu_ctx, oracle):
    n = k = 1536
    blocks = synth.q8_blocks(71, n, k)
    x = synth.normal_f32(72, k)
    w = q4.Q8Matrix.from_blocks(n, k, blocks, gpu_ctx)
    got = np.zeros(n, dtype=np.float32)
    q4.q8_apply(w, x, 1, got)
    assert_close(got, oracle.q8_apply(blocks, n, k, x, 1, threads=8), what="q8")
    w.free()
