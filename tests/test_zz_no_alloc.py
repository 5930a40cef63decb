"""lgh_q4_gemm_dev_noalloc, the entry point that allocates nothing, against lgh_q4_gemm_dev.

Named to be collected last: it must pass after every other GPU test as well as alone.

Both are called through the C ABI on the same device-resident inputs; the no-allocation variant
takes every scratch buffer from the device's fixed array, so its results must equal the
allocating entry point's bit for bit on every route (GEMV with x quantized once, dot4 batch with
codes, matrix-core batch, the GEMM with and without split-K, token chunks when the GEMM's scratch
exceeds the array), for two calls in a row on the shared array, the second with a smaller input.
"""

import ctypes as C

import numpy as np
import pytest

from llmhost_amd import _ffi, q4, synth

pytestmark = pytest.mark.gpu

SCRATCH = 32 << 20

# (n, k, first m, second m): the second call is smaller
CASES = [
    (8192, 16384, 1, 1),        # M=1 GEMV, x quantized once into scratch (K=16384 at N=8192)
    (1024, 4096, 4, 3),         # dot4 batch kernel on codes quantized once into scratch
    (2048, 2048, 16, 5),        # matrix-core batch kernel, activation image in scratch
    (10752, 2048, 512, 130),    # fp6 GEMM, no split
    (2048, 10752, 512, 100),    # fp6 GEMM with split-K partials in scratch
    (2048, 10752, 2048, 1100),  # GEMM whose 2048-token image exceeds the array: token chunks
    (512, 8192, 4096, 2100),    # chunks of fewer tiles keep the whole call's split count (none)
    (512, 65536, 1, 1),         # M=1 with K > 32768: the GEMM route
]


def _call(fn, ctx, w, x, y, m, mode):
    code = fn(ctx.handle, w.handle, C.c_void_p(x.data_ptr()), C.c_void_p(y.data_ptr()), m, mode)
    ctx.check(code)


@pytest.mark.parametrize("mode", [_ffi.LGH_ASSIGN, _ffi.LGH_ADD_F64])
@pytest.mark.parametrize("n,k,m1,m2", CASES)
def test_noalloc_equals_gemm_dev(gpu_ctx, n, k, m1, m2, mode):
    import torch

    print(f"[noalloc] n={n} k={k} m={m1},{m2} mode={mode}", flush=True)
    lib = _ffi.lib()
    w = q4.Q4Matrix.from_blocks(n, k, synth.q4_blocks(3001 + n + k, n, k), gpu_ctx)
    w.prepare_gemm()
    stream = torch.cuda.Stream()
    gpu_ctx.set_stream(stream.cuda_stream)
    try:
        with torch.cuda.stream(stream):
            for call, m in enumerate((m1, m2)):
                x = torch.from_numpy(synth.activations(3100 + call + m, m, k)).cuda()
                y0 = torch.from_numpy(synth.activations(3200 + call + m, m, n)).cuda()
                want, got = y0.clone(), y0.clone()
                _call(lib.lgh_q4_gemm_dev, gpu_ctx, w, x, want, m, mode)
                _call(lib.lgh_q4_gemm_dev_noalloc, gpu_ctx, w, x, got, m, mode)
                stream.synchronize()
                assert torch.equal(got, want), f"call {call}: m={m}"
                assert torch.isfinite(got).all()
    finally:
        gpu_ctx.set_stream(None)
        w.free()


def test_noalloc_needs_the_gemm_image(gpu_ctx):
    import torch

    n, k, m = 256, 2048, 128
    w = q4.Q4Matrix.from_blocks(n, k, synth.q4_blocks(3301, n, k), gpu_ctx)
    x = torch.zeros(m, k, device="cuda")
    y = torch.zeros(m, n, device="cuda")
    torch.cuda.synchronize()
    lib = _ffi.lib()
    with pytest.raises(q4.LghError, match="lgh_q4_prepare_gemm") as e:
        _call(lib.lgh_q4_gemm_dev_noalloc, gpu_ctx, w, x, y, m, _ffi.LGH_ASSIGN)
    assert e.value.code == _ffi.LGH_ERR_INVALID_ARG
    w.free()


def test_noalloc_rejects_scratch_beyond_the_array(gpu_ctx):
    """K = 655360: one 32-token activation image alone takes 34 MB > 32 MiB."""
    import torch

    n, k, m = 32, 655360, 65
    assert (k // 64) * 3328 * 1 > SCRATCH
    w = q4.Q4Matrix.from_blocks(n, k, synth.q4_blocks(3401, n, k), gpu_ctx)
    w.prepare_gemm()
    x = torch.zeros(m, k, device="cuda")
    y = torch.zeros(m, n, device="cuda")
    torch.cuda.synchronize()
    lib = _ffi.lib()
    with pytest.raises(q4.LghShapeError, match="fixed scratch"):
        _call(lib.lgh_q4_gemm_dev_noalloc, gpu_ctx, w, x, y, m, _ffi.LGH_ASSIGN)
    w.free()


def test_noalloc_rejects_mma_scratch_beyond_the_array(gpu_ctx):
    """40 tokens take the matrix-core batch route, whose activation image is taken in one piece:
    at K = 640000 it needs 3 token tiles x 5000 block quads x 2304 B = 34.6 MB > 32 MiB."""
    import torch

    n, k, m = 16, 640000, 40
    assert 3 * (k // 128) * (2048 + 256) > SCRATCH
    w = q4.Q4Matrix.from_blocks(n, k, synth.q4_blocks(3501, n, k), gpu_ctx)
    x = torch.zeros(m, k, device="cuda")
    y = torch.zeros(m, n, device="cuda")
    torch.cuda.synchronize()
    lib = _ffi.lib()
    with pytest.raises(q4.LghShapeError, match="fixed scratch"):
        _call(lib.lgh_q4_gemm_dev_noalloc, gpu_ctx, w, x, y, m, _ffi.LGH_ASSIGN)
    w.free()
