"""Behaviour of the C ABI around the kernels: stream ordering with torch, the GEMM image built on
first use, workspace growth under graph capture, lgh_trim."""

import numpy as np
import pytest

from llmhost_amd import _ffi, q4, synth

from .conftest import assert_close

pytestmark = pytest.mark.gpu


def _align(v):
    return (v + 255) // 256 * 256


def test_torch_stream_order(gpu_ctx, oracle):
    """x is written by a torch kernel queued behind slow work on torch's current stream, y is
    cleared by torch just before an AddF64 call, and y is read back by torch: with the library on
    its own stream, each call must still see torch's writes and torch must see the call's."""
    import torch

    n, k = 8192, 1536
    blocks = synth.q4_blocks(2101, n, k)
    xh = synth.normal_f32(2102, k)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    ref = oracle.gemv_q4(oracle.Q4Matrix(n, k, blocks), xh, threads=8)
    assert gpu_ctx.stream() != torch.cuda.current_stream().cuda_stream
    x_src = torch.from_numpy(xh).cuda()
    big = torch.randn(3072, 3072, device="cuda")
    torch.cuda.synchronize()
    for rep in range(3):
        x = torch.full((k,), float("nan"), device="cuda")
        y = torch.full((n,), float("nan"), device="cuda")
        for _ in range(6):  # slow work ahead of the writes on torch's stream
            big = torch.tanh(big @ big)
        x.copy_(x_src)
        q4.gemv_q4(w, x, y)
        assert_close(y.cpu().numpy(), ref, what=f"assign, rep {rep}")
        for _ in range(6):
            big = torch.tanh(big @ big)
        y.zero_()
        q4.gemv_q4_add(w, x, y)  # 0 + Wx in f64 == Wx
        assert_close(y.cpu().numpy(), ref, what=f"add, rep {rep}")
    w.free()


def test_gemm_image_built_on_first_gemm_use(gpu_ctx, oracle):
    """An upload holds only the 18 B / 32 planes; decode and small-batch routes never build the
    GEMM image; the first GEMM-route call builds it, and its results equal those of a matrix
    whose image was built up front."""
    import torch

    n, k = 640, 2048
    bpr = k // 32
    blocks = synth.q4_blocks(2201, n, k)
    planes = _align(n * bpr * 16) + _align(n * bpr * 2)
    image = ((n + 31) // 32) * ((bpr + 1) // 2) * 1792
    lazy = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    eager = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    assert lazy.device_bytes() == planes and eager.device_bytes() == planes
    eager.prepare_gemm()
    assert eager.device_bytes() == planes + image
    for m in (1, 4, 16, 64):  # GEMV, dot4 batch, matrix-core batch: no image
        x = synth.activations(2202 + m, m, k)
        y = np.zeros((m, n), dtype=np.float32)
        q4.gemm_q4(lazy, x, y, m)
        assert lazy.device_bytes() == planes, m
    m = 130
    x = synth.activations(2210, m, k)
    got, want = np.zeros((m, n), np.float32), np.zeros((m, n), np.float32)
    q4.gemm_q4(lazy, x, got, m)
    assert lazy.device_bytes() == planes + image
    q4.gemm_q4(eager, x, want, m)
    assert np.array_equal(got, want)
    assert_close(got, oracle.gemm_q4(oracle.Q4Matrix(n, k, blocks), x, m, threads=8), what="lazy image")
    # the device-pointer path builds it too
    lazy2 = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    yd = torch.zeros(m, n, device="cuda")
    q4.gemm_q4(lazy2, torch.from_numpy(x).cuda(), yd, m)
    assert np.array_equal(yd.cpu().numpy(), want)
    for w in (lazy, eager, lazy2):
        w.free()


def test_growth_under_capture_is_an_error_then_capture_after_warmup(gpu_ctx):
    """A call that would grow a workspace, or build a GEMM image, while its stream is being
    captured returns LGH_ERR_CAPTURE without enqueueing anything; after one eager call of the
    same shape the capture succeeds and every replay equals the eager result."""
    import torch

    ctx = q4.Context(0)  # fresh context: empty workspaces
    n, k, m = 2048, 2048, 256
    blocks = synth.q4_blocks(2301, n, k)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, ctx)
    stream = torch.cuda.Stream()
    ctx.set_stream(stream.cuda_stream)
    try:
        with torch.cuda.stream(stream):
            x = torch.from_numpy(synth.activations(2302, m, k)).cuda()
            y = torch.zeros(m, n, device="cuda")
            dummy = torch.zeros(1, device="cuda")
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            with pytest.raises(q4.LghError) as e1:
                q4.gemm_q4(w, x, y, m)  # no GEMM image yet
            dummy.add_(1.0)  # keep the captured graph non-empty
        assert e1.value.code == _ffi.LGH_ERR_CAPTURE
        del g
        w.prepare_gemm()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            with pytest.raises(q4.LghError) as e2:
                q4.gemm_q4(w, x, y, m)  # the workspace is still empty
            dummy.add_(1.0)
        assert e2.value.code == _ffi.LGH_ERR_CAPTURE
        del g
        with torch.cuda.stream(stream):
            q4.gemm_q4(w, x, y, m)  # eager: sizes the workspace
            eager = y.clone()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            q4.gemm_q4(w, x, y, m)
        for rep in range(3):
            with torch.cuda.stream(stream):
                y.fill_(float("nan"))
            g.replay()
            stream.synchronize()
            assert torch.equal(y, eager), rep
        del g
    finally:
        ctx.set_stream(None)
        w.free()
        ctx.close()


def test_trim_releases_workspaces_and_calls_still_work(gpu_ctx, oracle):
    n, k, m = 512, 1024, 100
    blocks = synth.q4_blocks(2401, n, k)
    x = synth.activations(2402, m, k)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    a, b = np.zeros((m, n), np.float32), np.zeros((m, n), np.float32)
    q4.gemm_q4(w, x, a, m)
    gpu_ctx.trim()
    q4.gemm_q4(w, x, b, m)
    assert np.array_equal(a, b)
    w.free()


def test_null_matrix_is_an_error_on_every_matrix_entry_point(gpu_ctx):
    """Each entry point that takes a matrix returns LGH_ERR_INVALID_ARG for a null one (the
    reference would not compile a missing matrix; here the check runs before any other argument
    is read, so the remaining pointers may be null too)."""
    L, h = _ffi.lib(), gpu_ctx.handle
    w = q4.Q4Matrix.from_blocks(64, 64, synth.q4_blocks(1, 64, 64), gpu_ctx)
    nul = None
    calls = {
        "lgh_q4_export": lambda: L.lgh_q4_export(h, nul, 0, nul, 0),
        "lgh_q8_export": lambda: L.lgh_q8_export(h, nul, nul, 0),
        "lgh_q4_prepare_gemm": lambda: L.lgh_q4_prepare_gemm(h, nul),
        "lgh_q4_gemv": lambda: L.lgh_q4_gemv(h, nul, nul, nul, 0),
        "lgh_q4_gemv_dev": lambda: L.lgh_q4_gemv_dev(h, nul, nul, nul, 0),
        "lgh_q4_gemv_pair (gate)": lambda: L.lgh_q4_gemv_pair(h, nul, w.handle, nul, nul, nul),
        "lgh_q4_gemv_pair (up)": lambda: L.lgh_q4_gemv_pair(h, w.handle, nul, nul, nul, nul),
        "lgh_q4_gemv_pair_dev": lambda: L.lgh_q4_gemv_pair_dev(h, nul, w.handle, nul, nul, nul),
        "lgh_q4_gemv_prep": lambda: L.lgh_q4_gemv_prep(h, nul, nul, nul, nul, 0),
        "lgh_q4_gemv_prep_dev": lambda: L.lgh_q4_gemv_prep_dev(h, nul, nul, nul, nul, 0),
        "lgh_q4_gemm": lambda: L.lgh_q4_gemm(h, nul, nul, nul, 4, 0),
        "lgh_q4_gemm_dev": lambda: L.lgh_q4_gemm_dev(h, nul, nul, nul, 4, 0),
        "lgh_q4_gemm_dev_noalloc": lambda: L.lgh_q4_gemm_dev_noalloc(h, nul, nul, nul, 4, 0),
        "lgh_q8_gemv": lambda: L.lgh_q8_gemv(h, nul, nul, nul, 1),
        "lgh_q8_gemv_dev": lambda: L.lgh_q8_gemv_dev(h, nul, nul, nul, 1),
        "lgh_q8_norm_gemv": lambda: L.lgh_q8_norm_gemv(h, nul, nul, 1e-5, nul, nul, 1),
        "lgh_q8_norm_gemv_dev": lambda: L.lgh_q8_norm_gemv_dev(h, nul, nul, 1e-5, nul, nul, 1),
        "lgh_q4_ffn_residual (w2)": lambda: L.lgh_q4_ffn_residual(h, w.handle, w.handle, nul, nul, 1e-5, nul, 1),
        "lgh_q4_ffn_residual (w1)": lambda: L.lgh_q4_ffn_residual(h, nul, w.handle, w.handle, nul, 1e-5, nul, 1),
        "lgh_q4_ffn_residual_dev (w3)": lambda: L.lgh_q4_ffn_residual_dev(h, w.handle, nul, w.handle, nul, 1e-5,
                                                                          nul, 1),
        "lgh_q4_mfma_block_dots": lambda: L.lgh_q4_mfma_block_dots(h, nul, nul, 1, nul),
    }
    try:
        for name, call in calls.items():
            assert call() == _ffi.LGH_ERR_INVALID_ARG, name
            assert b"null matrix" in L.lgh_last_error(h), name
        mats = (_ffi.C.c_void_p * 2)(w.handle, None)
        assert L.lgh_q4_norm_gemv(h, 2, mats, nul, 1e-5, nul, nul, 1, 0) == _ffi.LGH_ERR_INVALID_ARG
        assert b"null matrix 1" in L.lgh_last_error(h)
    finally:
        w.free()


@pytest.mark.parametrize("per_thread", [1, 2, 4, 8])
def test_probe_read_sums_what_it_reads(gpu_ctx, per_thread):
    """The streaming-read probe that benchmarks time beside the GEMVs reads every byte it is given:
    its per-workgroup sums match float64 sums of the same 4 KB * per_thread chunks (a ragged last
    chunk included), and the empty-kernel probe runs."""
    import torch

    print(f"[probe] per_thread={per_thread}", flush=True)
    nbytes = 7116800 + 48  # not a whole number of workgroup chunks
    src = torch.randn(nbytes // 4, device="cuda")
    nout = q4.probe_read_outputs(nbytes, per_thread)
    chunk = 256 * 16 * per_thread
    assert nout == (nbytes + chunk - 1) // chunk
    out = torch.full((nout + 1,), float("nan"), device="cuda")
    q4.probe_read(src, out, per_thread, gpu_ctx)
    q4.probe_empty(256, gpu_ctx)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    ref = np.add.reduceat(src.cpu().numpy().astype(np.float64), np.arange(0, nbytes // 4, chunk // 4))
    assert np.isnan(got[nout])  # nothing past the last workgroup's output
    np.testing.assert_allclose(got[:nout], ref, rtol=1e-5, atol=1e-3)
    with pytest.raises(q4.LghError):
        q4.probe_read(src, out, 3, gpu_ctx)
