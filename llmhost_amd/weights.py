"""Mirror of llm-engine's matmul seam (crates/llm-engine/src/weights.rs) on the GPU.

``Linear`` (weights.rs:11-103), ``apply_pair`` (weights.rs:106-123) and
``OutputHead`` (weights.rs:156-192) with the quantized variants dispatching to
libllm_gpu_hip.so instead of llm-cpu.  The fp32 variant of the reference
(``Linear::F32``) is not part of the block-quantized path and is not built.
"""

from __future__ import annotations

import numpy as np

from . import q4 as _q4
from ._ffi import LghShapeError, LGH_ERR_SHAPE
from .formats import BLOCK_SIZE


class LoadError(ValueError):
    """LoadError::Message (crates/llm-engine/src/load.rs)."""


class WeightFormat:
    """crates/llm-quant/src/formats.rs:9-57 (tags used on this path)."""

    Q8_0 = "Q8_0"
    Q4_32 = "Q4_32"


class Linear:
    """`Y = X @ W^T` with W [rows, cols] in Q4_32 (weights.rs:11-103)."""

    def __init__(self, mat: _q4.Q4Matrix):
        self.mat = mat

    @classmethod
    def from_f32(cls, weight: np.ndarray, rows: int, cols: int, fmt: str = WeightFormat.Q4_32,
                 ctx: _q4.Context | None = None) -> "Linear":
        """Linear::from_f32 (weights.rs:22-48)."""
        weight = np.asarray(weight, dtype=np.float32)
        if weight.size != rows * cols:
            raise LoadError(f"linear weight length {weight.size} != {rows}*{cols}")
        if fmt != WeightFormat.Q4_32:
            raise LoadError(f"unsupported linear weight format {fmt!r}")
        if cols % BLOCK_SIZE:
            raise LoadError(f"Q4 linear K={cols} is not a multiple of {BLOCK_SIZE}")
        return cls(_q4.Q4Matrix.from_f32(weight.ravel(), rows, cols, ctx))

    @classmethod
    def from_blocks(cls, blocks: np.ndarray, rows: int, cols: int, ctx: _q4.Context | None = None) -> "Linear":
        return cls(_q4.Q4Matrix.from_blocks(rows, cols, blocks, ctx))

    def rows(self) -> int:
        return self.mat.n

    def cols(self) -> int:
        return self.mat.k

    def _check(self, x, tokens: int, out) -> None:
        xs = x.numel() if hasattr(x, "numel") else x.size
        os_ = out.numel() if hasattr(out, "numel") else out.size
        if xs != tokens * self.cols() or os_ != tokens * self.rows():
            raise LghShapeError(LGH_ERR_SHAPE, "apply: x/out length mismatch (weights.rs:76-77)")

    def apply(self, x, tokens: int, out) -> None:
        """`out[tokens, rows] = x[tokens, cols] @ W^T` (weights.rs:75-88)."""
        self._check(x, tokens, out)
        if tokens == 1:
            _q4.gemv_q4(self.mat, x, out)
        else:
            _q4.gemm_q4(self.mat, x, out, tokens)

    def apply_add(self, x, tokens: int, dst) -> None:
        """`dst += x @ W^T` with the f64 residual add (weights.rs:91-102)."""
        self._check(x, tokens, dst)
        if tokens == 1:
            _q4.gemv_q4_add(self.mat, x, dst)
        else:
            _q4.gemm_q4_add(self.mat, x, dst, tokens)


def apply_pair(w1: Linear, w3: Linear, x, tokens: int, out1, out3) -> None:
    """SwiGLU gate (w1) and up (w3) sharing one activation (weights.rs:106-123)."""
    if tokens == 1 and w1.mat.n == w3.mat.n and w1.mat.k == w3.mat.k:
        _q4.gemv_q4_pair(w1.mat, w3.mat, x, out1, out3)
    else:
        w1.apply(x, tokens, out1)
        w3.apply(x, tokens, out3)


def norm_then_apply(linears, norm_w, eps: float, hidden, tokens: int, outs) -> None:
    """`normed = rms_norm(hidden)` then `linears[j].apply(normed, tokens, outs[j])` for 1..3 Q4
    linears sharing K: Lfm2::attn_decode's q/k/v (lfm2.rs:784-794) and conv_update's in_proj
    (lfm2.rs:651-659).  norm_w None: no norm.  One launch for a decode token with K <= 2048."""
    _q4.norm_gemv([lin.mat for lin in linears], norm_w, eps, hidden, outs, tokens)


def apply_then_add_inplace(linear: Linear, x, tokens: int, hidden) -> None:
    """`projected = linear.apply(x)` then `add_inplace(hidden, projected)` (ops.rs:48-53;
    lfm2.rs:645, 682, 749, 857): hidden += W x in f32, in one launch."""
    linear._check(x, tokens, hidden)
    _q4.apply_add_inplace(linear.mat, x, hidden, tokens)


class OutputHead:
    """Tied LM head, Q4 Linear or Q8_0 (weights.rs:156-192)."""

    def __init__(self, linear: Linear | None = None, q8: _q4.Q8Matrix | None = None):
        assert (linear is None) != (q8 is None)
        self.linear = linear
        self.q8 = q8

    @classmethod
    def from_embed(cls, embed: np.ndarray, vocab: int, hidden: int, fmt: str,
                   ctx: _q4.Context | None = None) -> "OutputHead":
        """OutputHead::from_embed (weights.rs:162-177)."""
        if fmt == WeightFormat.Q8_0:
            embed = np.asarray(embed, dtype=np.float32)
            if embed.size != vocab * hidden or hidden % BLOCK_SIZE:
                raise LoadError(f"Q8_0 head needs {vocab}*{hidden} values with hidden % 32 == 0")
            return cls(q8=_q4.Q8Matrix.from_f32(embed.ravel(), vocab, hidden, ctx))
        return cls(linear=Linear.from_f32(embed, vocab, hidden, fmt, ctx))

    def apply(self, x, tokens: int, out) -> None:
        if self.linear is not None:
            self.linear.apply(x, tokens, out)
        else:
            _q4.q8_apply(self.q8, x, tokens, out)

    def norm_apply(self, norm_w, eps: float, hidden, tokens: int, out) -> None:
        """`normed = rms_norm(hidden)` then `self.apply(normed)` (lfm2.rs:559-567, 496-504), the
        norm fused into the head's GEMV."""
        if self.linear is not None:
            _q4.norm_gemv([self.linear.mat], norm_w, eps, hidden, [out], tokens)
        else:
            _q4.q8_norm_apply(self.q8, norm_w, eps, hidden, tokens, out)
