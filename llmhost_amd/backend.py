"""Mirror of llm-core's Backend and Block traits for the HIP library.

``HipBackend`` is ``impl Backend`` (crates/llm-core/src/backend.rs:4-13, the CPU precedent at
crates/llm-cpu/src/lib.rs:65-75): ``name()`` is ``"hip"`` and ``alloc(len)`` returns a zeroed
device buffer of ``len`` f32 (``lgh_buffer_alloc``).  ``HipFfnBlock`` is ``impl Block``
(crates/llm-core/src/block.rs:6-14) for the FFN half of a layer: ``forward(input, output)``
writes ``output = input + W2 (silu(W1 n) * W3 n)`` with ``n = rms_norm(input)``
(``lgh_q4_ffn_residual``, crates/llm-engine/src/lfm2.rs:861-911).
"""

from __future__ import annotations

import ctypes as C
import enum

import numpy as np

from . import q4 as _q4
from ._ffi import LghShapeError, LGH_ERR_SHAPE, lib


class LayerKind(enum.Enum):
    """The two layer kinds of crates/llm-core/src/config.rs:35-48 (their parameters omitted)."""

    Conv = "conv"
    Attention = "attention"


class HipBuffer:
    """Backend::Buffer: `len` f32 in device memory, freed with lgh_buffer_free."""

    def __init__(self, ctx: _q4.Context, ptr: int, length: int):
        self.ctx = ctx
        self.ptr = ptr
        self.len = length

    def write(self, host: np.ndarray) -> None:
        host = np.ascontiguousarray(host, dtype=np.float32).ravel()
        if host.size != self.len:
            raise LghShapeError(LGH_ERR_SHAPE, f"buffer holds {self.len} floats, got {host.size}")
        self.ctx.check(lib().lgh_buffer_write(self.ctx.handle, C.c_void_p(self.ptr), host.ctypes.data_as(C.c_void_p),
                                              self.len))

    def read(self) -> np.ndarray:
        out = np.empty(self.len, dtype=np.float32)
        self.ctx.check(lib().lgh_buffer_read(self.ctx.handle, out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr),
                                             self.len))
        return out

    def free(self) -> None:
        if self.ptr:
            lib().lgh_buffer_free(self.ctx.handle, C.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HipBackend:
    """impl Backend for the HIP library (backend.rs:4-13)."""

    def __init__(self, ctx: _q4.Context | None = None):
        self.ctx = ctx or _q4.default_context()

    def name(self) -> str:
        return "hip"

    def alloc(self, length: int) -> HipBuffer:
        p = C.c_void_p()
        self.ctx.check(lib().lgh_buffer_alloc(self.ctx.handle, length, C.byref(p)))
        return HipBuffer(self.ctx, p.value or 0, length)


class HipFfnBlock:
    """impl Block (block.rs:6-14) for the FFN half of a layer of kind `kind`."""

    def __init__(self, kind: LayerKind, w1: _q4.Q4Matrix, w3: _q4.Q4Matrix, w2: _q4.Q4Matrix, norm_w, eps: float):
        if not (w1.k == w3.k == w2.n and w1.n == w3.n == w2.k):
            raise LghShapeError(LGH_ERR_SHAPE, "FFN shapes: W1, W3 [inter, dim], W2 [dim, inter]")
        self._kind = kind
        self.w1, self.w3, self.w2 = w1, w3, w2
        self.norm_w = np.ascontiguousarray(norm_w, dtype=np.float32)
        self.eps = float(eps)

    def kind(self) -> LayerKind:
        return self._kind

    def forward(self, input: np.ndarray, output: np.ndarray) -> None:
        """output = input + FFN(rms_norm(input)) over input.size / dim token rows."""
        dim = self.w1.k
        _q4._host_f32(output, "output")
        if input.size != output.size or input.size % dim:
            raise LghShapeError(LGH_ERR_SHAPE, f"forward: input {input.size} / output {output.size} floats, "
                                               f"dim {dim}")
        np.copyto(output, input)
        _q4.ffn_residual(self.w1, self.w3, self.w2, self.norm_w, self.eps, output.reshape(-1), input.size // dim)
