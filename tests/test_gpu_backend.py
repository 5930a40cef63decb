"""The Backend / Block mirror (crates/llm-core/src/backend.rs:4-13, block.rs:6-14) through the C ABI:
device buffers from lgh_buffer_alloc (zeroed, like CpuBackend::alloc), host round trips, and one
forward of the HIP FFN block against the oracle's ffn_residual."""

import ctypes as C

import numpy as np
import pytest

from llmhost_amd import _ffi, q4, synth
from llmhost_amd.backend import HipBackend, HipFfnBlock, LayerKind

from .conftest import assert_close

pytestmark = pytest.mark.gpu


def test_backend_alloc_is_zeroed_and_round_trips(gpu_ctx):
    be = HipBackend(gpu_ctx)
    assert be.name() == "hip"
    for n in (1, 37, 1 << 20):
        buf = be.alloc(n)
        assert buf.ptr and buf.len == n
        assert not buf.read().any()
        data = synth.normal_f32(n, n)
        buf.write(data)
        assert np.array_equal(buf.read(), data)
        buf.free()
    empty = be.alloc(0)
    assert empty.ptr == 0 and empty.read().size == 0


def test_backend_buffer_feeds_the_dev_entry_points(gpu_ctx, oracle):
    """A Backend buffer is a plain device pointer for the *_dev calls (here lgh_q4_gemv_dev)."""
    n, k = 1024, 1536
    blocks = synth.q4_blocks(4001, n, k)
    w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
    be = HipBackend(gpu_ctx)
    xb, yb = be.alloc(k), be.alloc(n)
    x = synth.normal_f32(4002, k)
    xb.write(x)
    lib = _ffi.lib()
    gpu_ctx.check(lib.lgh_q4_gemv_dev(gpu_ctx.handle, w.handle, C.c_void_p(xb.ptr), C.c_void_p(yb.ptr),
                                      _ffi.LGH_ASSIGN))
    assert_close(yb.read(), oracle.gemv_q4(oracle.Q4Matrix(n, k, blocks), x, threads=8), what="gemv via buffers")
    xb.free()
    yb.free()
    w.free()


@pytest.mark.parametrize("tokens", [1, 3])
def test_ffn_block_forward(gpu_ctx, oracle, tokens):
    dim, inter = 1536, 8192
    bl = [synth.q4_blocks(4100 + j, n, k) for j, (n, k) in enumerate([(inter, dim), (inter, dim), (dim, inter)])]
    w1, w3, w2 = (q4.Q4Matrix.from_blocks(b.size * 32 // k, k, b, gpu_ctx)
                  for b, k in zip(bl, (dim, dim, inter)))
    nw = (1 + 0.1 * synth.normal_f32(4110, dim)).astype(np.float32)
    block = HipFfnBlock(LayerKind.Attention, w1, w3, w2, nw, 1e-5)
    assert block.kind() is LayerKind.Attention
    x = synth.activations(4111 + tokens, tokens, dim)
    out = np.zeros_like(x)
    block.forward(x, out)
    want = x.copy().ravel()
    q4.ffn_residual(w1, w3, w2, nw, 1e-5, want, tokens)
    assert np.array_equal(out.ravel(), want)  # forward == the block's entry point on a copy of input
    assert not np.array_equal(out, x)
    with pytest.raises(q4.LghShapeError):
        block.forward(x, np.zeros((tokens, dim + 32), np.float32))
    for w in (w1, w3, w2):
        w.free()
