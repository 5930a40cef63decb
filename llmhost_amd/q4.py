"""Host-side mirror of llm-cpu's quantized-matmul API on the HIP library.

Same names, argument meaning and error behaviour as the reference functions
(crates/llm-cpu/src/gemv_q4.rs, re-exported at crates/llm-cpu/src/lib.rs:21-24),
with the computation done by libllm_gpu_hip.so on one MI355X:

    Q4Matrix.from_blocks(n, k, blocks) / Q4Matrix.from_f32(w, n, k)
    gemv_q4(w, x, out) / gemv_q4_add(w, x, dst) / gemv_q4_pair(wg, wu, x, og, ou)
    gemm_q4(w, x, out, m) / gemm_q4_add(w, x, out, m)
    ActQ8.quantize(x) / ActQ8.quantize_row(x)
    set_act_quant(ActQuant.PerRow) / current_act_quant()
    Q8Matrix + q8_apply (crates/llm-engine/src/weights.rs:126-227)

Operands are numpy arrays (host memory, synchronous, like the reference's
slices) or torch tensors on the GPU (device memory, enqueued on the
context's stream).  A call on torch tensors is ordered after the work already
queued on torch's current stream, and torch's current stream is ordered after
the call, so the kernels read what torch wrote before the call and torch reads
what they wrote.  Where the reference `assert!`s (length mismatch,
k % 32 != 0) these raise ``LghShapeError`` (a ValueError) and write nothing.

A process-wide default context (device 0) plays the role of llm-cpu's
process-wide state; ``Context`` objects can be passed explicitly instead.
"""

from __future__ import annotations

import ctypes as C
import enum
import threading

import numpy as np

from . import _ffi
from ._ffi import LghError, LghShapeError, check, lib
from .formats import BLOCK_Q4, BLOCK_Q8_0, BLOCK_SIZE


class ActQuant(enum.IntEnum):
    """gemv_q4.rs:263-271."""

    PerBlock = _ffi.LGH_ACT_PER_BLOCK
    PerRow = _ffi.LGH_ACT_PER_ROW


class Context:
    """An lgh_ctx: one device, one stream, workspaces, act-quant mode."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        code = lib().lgh_init(device, C.byref(h))
        if code != _ffi.LGH_OK:
            raise _ffi.LghError(code, lib().lgh_last_error(None).decode())
        self.handle = h
        self.device = device
        self._stream_handle = lib().lgh_get_stream(h) or 0
        self._torch_stream = None  # torch view of the context stream, made on first use

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().lgh_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, code: int) -> None:
        check(code, self.handle)

    def set_act_quant(self, mode: ActQuant) -> None:
        self.check(lib().lgh_set_act_quant(self.handle, int(mode)))

    def act_quant(self) -> ActQuant:
        return ActQuant(lib().lgh_get_act_quant(self.handle))

    def set_stream(self, stream_handle: int | None) -> None:
        """Use a hipStream_t (e.g. torch.cuda.current_stream().cuda_stream)."""
        self.check(lib().lgh_set_stream(self.handle, C.c_void_p(stream_handle or 0)))
        self._stream_handle = lib().lgh_get_stream(self.handle) or 0
        self._torch_stream = None

    def stream(self) -> int:
        return self._stream_handle

    def trim(self) -> None:
        """lgh_trim: release the context's workspaces (they grow again when needed)."""
        self.check(lib().lgh_trim(self.handle))

    def dev_call(self, launch) -> None:
        """Run `launch` (which enqueues on the context stream) in torch's stream order: the context
        stream first waits for torch's current stream, and torch's current stream then waits for
        the context stream.  No waits when the two are the same stream."""
        import torch

        cur = torch.cuda.current_stream(self.device)
        if cur.cuda_stream == self._stream_handle:
            launch()
            return
        if self._torch_stream is None:
            self._torch_stream = torch.cuda.ExternalStream(self._stream_handle, device=self.device)
        ext = self._torch_stream
        ext.wait_stream(cur)
        try:
            launch()
        finally:
            cur.wait_stream(ext)

    def sync(self) -> None:
        self.check(lib().lgh_sync(self.handle))


_default_ctx: Context | None = None
_default_lock = threading.Lock()


def default_context() -> Context:
    global _default_ctx
    with _default_lock:
        if _default_ctx is None:
            _default_ctx = Context(0)
        return _default_ctx


def set_act_quant(mode: ActQuant, ctx: Context | None = None) -> None:
    """set_act_quant (gemv_q4.rs:276-282), per context."""
    (ctx or default_context()).set_act_quant(mode)


def current_act_quant(ctx: Context | None = None) -> ActQuant:
    """current_act_quant (gemv_q4.rs:286-292)."""
    return (ctx or default_context()).act_quant()


# ---- operand plumbing ------------------------------------------------------
def _is_torch(a) -> bool:
    return type(a).__module__.startswith("torch")


def _host_f32(a, name: str) -> np.ndarray:
    if not isinstance(a, np.ndarray) or a.dtype != np.float32 or not a.flags["C_CONTIGUOUS"]:
        raise TypeError(f"{name} must be a C-contiguous float32 numpy array")
    return a


def _dev_ptr(a, name: str) -> C.c_void_p:
    import torch

    if a.device.type != "cuda" or a.dtype != torch.float32 or not a.is_contiguous():
        raise TypeError(f"{name} must be a contiguous float32 tensor on the GPU")
    return C.c_void_p(a.data_ptr())


def _dev_ptr_of(a, name: str, dtype) -> C.c_void_p:
    """Device pointer of a contiguous tensor of `dtype` on the GPU."""
    if a.device.type != "cuda" or a.dtype != dtype or not a.is_contiguous():
        raise TypeError(f"{name} must be a contiguous {dtype} tensor on the GPU")
    return C.c_void_p(a.data_ptr())


def _np_ptr(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


def _shape_assert(cond: bool, msg: str) -> None:
    if not cond:
        raise LghShapeError(_ffi.LGH_ERR_SHAPE, msg)


def _check_norm_w(norm_w, k: int) -> None:
    """rms_norm asserts weight.len() == dim (crates/llm-cpu/src/ops.rs:9-11); the library reads k
    floats of the norm weight, so a shorter one must never reach it."""
    if norm_w is None:
        return
    size = norm_w.numel() if _is_torch(norm_w) else np.asarray(norm_w).size
    _shape_assert(size == k, f"norm weight length {size} != {k}")


# ---- matrices -----------------------------------------------------------------
class Q4Matrix:
    """Device-resident Q4 matrix [n, k] (gemv_q4.rs:97-209)."""

    def __init__(self, handle: C.c_void_p, n: int, k: int, ctx: Context):
        self._h = handle
        self.n = n
        self.k = k
        self.ctx = ctx

    @classmethod
    def from_blocks(cls, n: int, k: int, blocks: np.ndarray, ctx: Context | None = None) -> "Q4Matrix":
        """Q4Matrix::from_blocks (gemv_q4.rs:128-149)."""
        ctx = ctx or default_context()
        _shape_assert(k % BLOCK_SIZE == 0, f"K={k} is not a multiple of {BLOCK_SIZE}")
        h = C.c_void_p()
        if _is_torch(blocks):
            _shape_assert(blocks.numel() * blocks.element_size() == n * (k // 32) * 18,
                          "blocks byte length != n*k/32*18")
            ctx.dev_call(lambda: ctx.check(
                lib().lgh_q4_upload_dev(ctx.handle, C.c_void_p(blocks.data_ptr()), n, k, C.byref(h))))
        else:
            blocks = np.ascontiguousarray(blocks)
            _shape_assert(blocks.dtype == BLOCK_Q4 and blocks.size == n * (k // 32),
                          f"expected {n * (k // 32)} BlockQ4 blocks")
            ctx.check(lib().lgh_q4_upload(ctx.handle, _np_ptr(blocks), n, k, C.byref(h)))
        return cls(h, n, k, ctx)

    @classmethod
    def from_f32(cls, weight: np.ndarray, n: int, k: int, ctx: Context | None = None) -> "Q4Matrix":
        """Q4Matrix::from_f32 (gemv_q4.rs:116-124): BlockQ4::quantize on the GPU."""
        ctx = ctx or default_context()
        w = _host_f32(np.ascontiguousarray(weight, dtype=np.float32), "weight")
        _shape_assert(w.size == n * k, f"weight length {w.size} != {n}*{k}")
        _shape_assert(k % BLOCK_SIZE == 0, f"K={k} is not a multiple of {BLOCK_SIZE}")
        h = C.c_void_p()
        ctx.check(lib().lgh_q4_from_f32(ctx.handle, _np_ptr(w), n, k, C.byref(h)))
        return cls(h, n, k, ctx)

    def blocks(self) -> np.ndarray:
        """The matrix as row-major BlockQ4[n][k/32] (as uploaded)."""
        out = np.zeros(self.n * (self.k // 32), dtype=BLOCK_Q4)
        self.ctx.check(lib().lgh_q4_download(self.ctx.handle, self._h, _np_ptr(out)))
        return out

    def blocks_per_row(self) -> int:
        return self.k // BLOCK_SIZE

    def prepare_gemm(self) -> None:
        """lgh_q4_prepare_gemm: build the GEMM operand image now instead of on first GEMM use."""
        self.ctx.check(lib().lgh_q4_prepare_gemm(self.ctx.handle, self._h))

    def device_bytes(self) -> int:
        """Device bytes held: nibble and scale planes, plus the GEMM image once built."""
        return int(lib().lgh_q4_device_bytes(self._h))

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def free(self) -> None:
        if getattr(self, "_h", None):
            lib().lgh_q4_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Q8Matrix:
    """Device-resident Q8_0 matrix (crates/llm-engine/src/weights.rs:126-153)."""

    def __init__(self, handle: C.c_void_p, n: int, k: int, ctx: Context):
        self._h = handle
        self.n = n
        self.k = k
        self.ctx = ctx

    @classmethod
    def from_blocks(cls, n: int, k: int, blocks: np.ndarray, ctx: Context | None = None) -> "Q8Matrix":
        ctx = ctx or default_context()
        _shape_assert(k % BLOCK_SIZE == 0, f"K={k} is not a multiple of {BLOCK_SIZE}")
        blocks = np.ascontiguousarray(blocks)
        _shape_assert(blocks.dtype == BLOCK_Q8_0 and blocks.size == n * (k // 32),
                      f"expected {n * (k // 32)} BlockQ8_0 blocks")
        h = C.c_void_p()
        ctx.check(lib().lgh_q8_upload(ctx.handle, _np_ptr(blocks), n, k, C.byref(h)))
        return cls(h, n, k, ctx)

    @classmethod
    def from_f32(cls, weight: np.ndarray, n: int, k: int, ctx: Context | None = None) -> "Q8Matrix":
        """Q8Matrix::from_f32 (weights.rs:133-142): BlockQ8_0::quantize on the GPU."""
        ctx = ctx or default_context()
        w = _host_f32(np.ascontiguousarray(weight, dtype=np.float32), "weight")
        _shape_assert(w.size == n * k, f"weight length {w.size} != {n}*{k}")
        _shape_assert(k % BLOCK_SIZE == 0, f"K={k} is not a multiple of {BLOCK_SIZE}")
        h = C.c_void_p()
        ctx.check(lib().lgh_q8_from_f32(ctx.handle, _np_ptr(w), n, k, C.byref(h)))
        return cls(h, n, k, ctx)

    def blocks(self) -> np.ndarray:
        out = np.zeros(self.n * (self.k // 32), dtype=BLOCK_Q8_0)
        self.ctx.check(lib().lgh_q8_download(self.ctx.handle, self._h, _np_ptr(out)))
        return out

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def free(self) -> None:
        if getattr(self, "_h", None):
            lib().lgh_q8_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---- activation quant ----------------------------------------------------------
class ActQ8:
    """ActQ8 (gemv_q4.rs:25-95) computed by the device act-quant kernel."""

    def __init__(self, qs: np.ndarray, scales: np.ndarray, sums: np.ndarray):
        self.qs = qs
        self.scales = scales
        self.sums = sums

    @classmethod
    def _run(cls, x, mode: ActQuant, ctx: Context | None) -> "ActQ8":
        ctx = ctx or default_context()
        if _is_torch(x):
            return cls._run_dev(x, mode, ctx)
        x = _host_f32(np.ascontiguousarray(x, dtype=np.float32), "x")
        k = x.shape[-1]
        _shape_assert(k % BLOCK_SIZE == 0, f"activation length {k} is not a multiple of {BLOCK_SIZE}")
        m = x.size // k if k else 0
        qs = np.zeros(x.shape, dtype=np.int8)
        sc = np.zeros(x.shape[:-1] + (k // 32,), dtype=np.float32)
        su = np.zeros(x.shape[:-1] + (k // 32,), dtype=np.int32)
        prev = ctx.act_quant()
        ctx.set_act_quant(mode)
        try:
            ctx.check(lib().lgh_act_quant(ctx.handle, _np_ptr(x), m, k, _np_ptr(qs), _np_ptr(sc), _np_ptr(su)))
        finally:
            ctx.set_act_quant(prev)
        return cls(qs, sc, su)

    @classmethod
    def _run_dev(cls, x, mode: ActQuant, ctx: Context) -> "ActQ8":
        """Device tensors in and out, enqueued on the context stream (lgh_act_quant_dev)."""
        import torch

        k = x.shape[-1]
        _shape_assert(k % BLOCK_SIZE == 0, f"activation length {k} is not a multiple of {BLOCK_SIZE}")
        m = x.numel() // k if k else 0
        qs = torch.zeros(x.shape, dtype=torch.int8, device=x.device)
        sc = torch.zeros(x.shape[:-1] + (k // 32,), dtype=torch.float32, device=x.device)
        su = torch.zeros(x.shape[:-1] + (k // 32,), dtype=torch.int32, device=x.device)
        prev = ctx.act_quant()
        ctx.set_act_quant(mode)
        try:
            ctx.dev_call(lambda: ctx.check(lib().lgh_act_quant_dev(
                ctx.handle, _dev_ptr(x, "x"), m, k, _dev_ptr_of(qs, "qs", torch.int8),
                _dev_ptr_of(sc, "scales", torch.float32), _dev_ptr_of(su, "sums", torch.int32))))
        finally:
            ctx.set_act_quant(prev)
        return cls(qs, sc, su)

    @classmethod
    def quantize(cls, x, ctx: Context | None = None) -> "ActQ8":
        """ActQ8::quantize (gemv_q4.rs:35-40): per-block scales."""
        return cls._run(x, ActQuant.PerBlock, ctx)

    @classmethod
    def quantize_row(cls, x, ctx: Context | None = None) -> "ActQ8":
        """ActQ8::quantize_row (gemv_q4.rs:44-49): one scale per row."""
        return cls._run(x, ActQuant.PerRow, ctx)


# ---- GEMV / GEMM ----------------------------------------------------------------
def _gemm(w: Q4Matrix, x, out, m: int, mode: int) -> None:
    ctx = w.ctx
    if _is_torch(x) or _is_torch(out):
        _shape_assert(x.numel() == m * w.k, f"x length {x.numel()} != {m}*{w.k}")
        _shape_assert(out.numel() == m * w.n, f"out length {out.numel()} != {m}*{w.n}")
        xp, op = _dev_ptr(x, "x"), _dev_ptr(out, "out")
        ctx.dev_call(lambda: ctx.check(lib().lgh_q4_gemm_dev(ctx.handle, w.handle, xp, op, m, mode)))
        return
    x = _host_f32(x, "x")
    out = _host_f32(out, "out")
    _shape_assert(x.size == m * w.k, f"x length {x.size} != {m}*{w.k}")
    _shape_assert(out.size == m * w.n, f"out length {out.size} != {m}*{w.n}")
    ctx.check(lib().lgh_q4_gemm(ctx.handle, w.handle, _np_ptr(x), _np_ptr(out), m, mode))


def probe_empty(workgroups: int = 1, ctx: Context | None = None) -> None:
    """One launch of an empty kernel of `workgroups` x 256 threads (lgh_probe_empty_dev), in torch's
    stream order: the per-launch floor a benchmark times beside the matmuls."""
    ctx = ctx or default_context()
    ctx.dev_call(lambda: ctx.check(lib().lgh_probe_empty_dev(ctx.handle, int(workgroups))))


def probe_read(src, out, per_thread: int = 4, ctx: Context | None = None) -> None:
    """A plain streaming read of the device tensor `src` (lgh_probe_read_dev): one f32 sum per
    workgroup into the device tensor `out` (``probe_read_outputs`` floats)."""
    ctx = ctx or default_context()
    nbytes = src.numel() * src.element_size()
    need = probe_read_outputs(nbytes, per_thread)
    sp, op = _dev_ptr_of(src, "src", src.dtype), _dev_ptr(out, "out")
    _shape_assert(out.numel() >= need, f"out holds {out.numel()} floats, the read writes {need}")
    ctx.dev_call(lambda: ctx.check(lib().lgh_probe_read_dev(ctx.handle, sp, nbytes, int(per_thread), op)))


def probe_read_outputs(nbytes: int, per_thread: int = 4) -> int:
    return int(lib().lgh_probe_read_outputs(nbytes, int(per_thread)))


def gemv_q4(w: Q4Matrix, x, out) -> None:
    """`out[n] = W[n, k] @ x[k]` with on-the-fly Q8 activations (gemv_q4.rs:344-352)."""
    _gemm(w, x, out, 1, _ffi.LGH_ASSIGN)


def gemv_q4_add(w: Q4Matrix, x, dst) -> None:
    """Adds the product onto dst in f64 (gemv_q4.rs:355-363)."""
    _gemm(w, x, dst, 1, _ffi.LGH_ADD_F64)


def _gemv_prep(w: Q4Matrix, acts: ActQ8, out, mode: int) -> None:
    ctx = w.ctx
    if _is_torch(acts.qs) or _is_torch(out):
        import torch

        _shape_assert(acts.qs.numel() == w.k, f"acts length {acts.qs.numel()} != {w.k}")
        _shape_assert(acts.scales.numel() == w.k // 32, f"acts scales {acts.scales.numel()} != {w.k // 32}")
        _shape_assert(out.numel() == w.n, f"out length {out.numel()} != {w.n}")
        qp = _dev_ptr_of(acts.qs, "acts.qs", torch.int8)
        sp = _dev_ptr_of(acts.scales, "acts.scales", torch.float32)
        op = _dev_ptr(out, "out")
        ctx.dev_call(lambda: ctx.check(lib().lgh_q4_gemv_prep_dev(ctx.handle, w.handle, qp, sp, op, mode)))
        return
    qs = np.ascontiguousarray(acts.qs, dtype=np.int8)
    sc = _host_f32(np.ascontiguousarray(acts.scales, dtype=np.float32), "acts.scales")
    out = _host_f32(out, "out")
    _shape_assert(qs.size == w.k, f"acts length {qs.size} != {w.k}")
    _shape_assert(sc.size == w.k // 32, f"acts scales {sc.size} != {w.k // 32}")
    _shape_assert(out.size == w.n, f"out length {out.size} != {w.n}")
    ctx.check(lib().lgh_q4_gemv_prep(ctx.handle, w.handle, _np_ptr(qs), _np_ptr(sc), _np_ptr(out), mode))


def gemv_q4_prep(w: Q4Matrix, acts: ActQ8, out) -> None:
    """GEMV on already-quantized activations (gemv_q4.rs:366-378)."""
    _gemv_prep(w, acts, out, _ffi.LGH_ASSIGN)


def gemv_q4_prep_add(w: Q4Matrix, acts: ActQ8, dst) -> None:
    """Fused add variant of gemv_q4_prep (gemv_q4.rs:380-393)."""
    _gemv_prep(w, acts, dst, _ffi.LGH_ADD_F64)


def gemm_q4(w: Q4Matrix, x, out, m: int) -> None:
    """Prefill `out[m, n] = X[m, k] @ W[n, k]^T` (gemv_q4.rs:686-688)."""
    _gemm(w, x, out, m, _ffi.LGH_ASSIGN)


def gemm_q4_add(w: Q4Matrix, x, out, m: int) -> None:
    """Like gemm_q4 but adds onto out in f64 (gemv_q4.rs:691-693)."""
    _gemm(w, x, out, m, _ffi.LGH_ADD_F64)


def apply_add_inplace(w: Q4Matrix, x, dst, m: int = 1) -> None:
    """`dst += X @ W^T` in f32, one launch: Linear::apply into a scratch then ops::add_inplace
    (crates/llm-cpu/src/ops.rs:48-53), the residual step after an attention or conv block's
    out_proj (crates/llm-engine/src/lfm2.rs:645, 682, 749, 857)."""
    _gemm(w, x, dst, m, _ffi.LGH_ADD_F32)


def gemv_q4_pair(w_gate: Q4Matrix, w_up: Q4Matrix, x, out_gate, out_up) -> None:
    """Gate and up GEMVs sharing one activation quant (gemv_q4.rs:396-443)."""
    ctx = w_gate.ctx
    _shape_assert(w_gate.k == w_up.k, "gate/up K differ")
    _shape_assert(w_gate.n == w_up.n, "gate/up N differ")
    if _is_torch(x):
        _shape_assert(x.numel() == w_gate.k, "x length != K")
        _shape_assert(out_gate.numel() == w_gate.n and out_up.numel() == w_up.n, "out length != N")
        xp, gp, up = _dev_ptr(x, "x"), _dev_ptr(out_gate, "out_gate"), _dev_ptr(out_up, "out_up")
        ctx.dev_call(lambda: ctx.check(
            lib().lgh_q4_gemv_pair_dev(ctx.handle, w_gate.handle, w_up.handle, xp, gp, up)))
        return
    x = _host_f32(x, "x")
    out_gate = _host_f32(out_gate, "out_gate")
    out_up = _host_f32(out_up, "out_up")
    _shape_assert(x.size == w_gate.k, "x length != K")
    _shape_assert(out_gate.size == w_gate.n and out_up.size == w_up.n, "out length != N")
    ctx.check(lib().lgh_q4_gemv_pair(ctx.handle, w_gate.handle, w_up.handle, _np_ptr(x), _np_ptr(out_gate),
                                     _np_ptr(out_up)))


# ---- FFN block ---------------------------------------------------------------
def rms_norm(x, weight, eps: float, out, ctx: Context | None = None) -> None:
    """rms_norm (crates/llm-cpu/src/ops.rs:8-23) over the rows of x (row length = weight size)."""
    ctx = ctx or default_context()
    if _is_torch(x):
        _shape_assert(weight.numel() > 0 and x.numel() % weight.numel() == 0 and out.numel() == x.numel(),
                      "rms_norm shapes")
        xp, wp, op = _dev_ptr(x, "x"), _dev_ptr(weight, "weight"), _dev_ptr(out, "out")
        ctx.dev_call(lambda: ctx.check(lib().lgh_rms_norm_dev(ctx.handle, xp, wp, weight.numel(),
                                                              x.numel() // weight.numel(), float(eps), op)))
        return
    x, weight, out = _host_f32(x, "x"), _host_f32(weight, "weight"), _host_f32(out, "out")
    _shape_assert(weight.size > 0 and x.size % weight.size == 0 and out.size == x.size, "rms_norm shapes")
    ctx.check(lib().lgh_rms_norm(ctx.handle, _np_ptr(x), _np_ptr(weight), weight.size, x.size // weight.size,
                                 float(eps), _np_ptr(out)))


def silu_mul(g, u, ctx: Context | None = None) -> None:
    """g = silu(g) * u in place (ops.rs:27-36, lfm2.rs:902-905)."""
    ctx = ctx or default_context()
    if _is_torch(g):
        _shape_assert(g.numel() == u.numel(), "g/u lengths differ")
        gp, up = _dev_ptr(g, "g"), _dev_ptr(u, "u")
        ctx.dev_call(lambda: ctx.check(lib().lgh_silu_mul_dev(ctx.handle, gp, up, g.numel())))
        return
    g, u = _host_f32(g, "g"), _host_f32(u, "u")
    _shape_assert(g.size == u.size, "g/u lengths differ")
    ctx.check(lib().lgh_silu_mul(ctx.handle, _np_ptr(g), _np_ptr(u), g.size))


def ffn_residual(w1: Q4Matrix, w3: Q4Matrix, w2: Q4Matrix, norm_w, eps: float, hidden, tokens: int = 1) -> None:
    """Lfm2::ffn_residual / ffn_residual_in (crates/llm-engine/src/lfm2.rs:861-911) over `tokens`
    rows: hidden += W2 (silu(W1 n) * W3 n) with n = rms_norm(hidden, norm_w, eps) (norm_w None:
    n = hidden); the down projection is added in f64.  hidden is updated in place (numpy or
    torch)."""
    ctx = w1.ctx
    _shape_assert(w1.k == w3.k == w2.n and w1.n == w3.n == w2.k, "FFN shapes: W1, W3 [inter, dim], W2 [dim, inter]")
    _check_norm_w(norm_w, w1.k)
    if _is_torch(hidden):
        _shape_assert(hidden.numel() == tokens * w1.k, "hidden length != tokens * dim")
        nw = None if norm_w is None else _dev_ptr(norm_w, "norm_w")
        hp = _dev_ptr(hidden, "hidden")
        ctx.dev_call(lambda: ctx.check(lib().lgh_q4_ffn_residual_dev(ctx.handle, w1.handle, w3.handle, w2.handle,
                                                                     nw, float(eps), hp, tokens)))
        return
    hidden = _host_f32(hidden, "hidden")
    _shape_assert(hidden.size == tokens * w1.k, "hidden length != tokens * dim")
    nw = None if norm_w is None else _np_ptr(_host_f32(norm_w, "norm_w"))
    ctx.check(lib().lgh_q4_ffn_residual(ctx.handle, w1.handle, w3.handle, w2.handle, nw, float(eps),
                                        _np_ptr(hidden), tokens))


def norm_gemv(ws, norm_w, eps: float, hidden, outs, tokens: int = 1, mode: int = _ffi.LGH_ASSIGN) -> None:
    """rms_norm of `tokens` rows of hidden, then outs[j] = W[j] normed for 1..3 matrices with the
    same K: the q/k/v projections of Lfm2::attn_decode (crates/llm-engine/src/lfm2.rs:784-794) or
    the in_proj of Lfm2::conv_update (lfm2.rs:651-659).  norm_w None: no norm.  One token with
    K <= 2048 is one launch sharing one activation quantization; numpy or torch operands."""
    ws = list(ws)
    outs = list(outs)
    _shape_assert(1 <= len(ws) <= 3 and len(outs) == len(ws), "1 to 3 matrices, one output each")
    ctx = ws[0].ctx
    k = ws[0].k
    _shape_assert(all(w.k == k for w in ws), "matrices must share K")
    _check_norm_w(norm_w, k)
    handles = (C.c_void_p * len(ws))(*[w.handle.value for w in ws])
    if _is_torch(hidden):
        _shape_assert(hidden.numel() == tokens * k, "hidden length != tokens * K")
        _shape_assert(all(o.numel() == tokens * w.n for o, w in zip(outs, ws)), "out length != tokens * N")
        ptrs = (C.c_void_p * len(ws))(*[_dev_ptr(o, "out").value for o in outs])
        nw = None if norm_w is None else _dev_ptr(norm_w, "norm_w")
        hp = _dev_ptr(hidden, "hidden")
        ctx.dev_call(lambda: ctx.check(lib().lgh_q4_norm_gemv_dev(ctx.handle, len(ws), handles, nw, float(eps), hp,
                                                                  ptrs, tokens, mode)))
        return
    hidden = _host_f32(hidden, "hidden")
    outs = [_host_f32(o, "out") for o in outs]
    _shape_assert(hidden.size == tokens * k, "hidden length != tokens * K")
    _shape_assert(all(o.size == tokens * w.n for o, w in zip(outs, ws)), "out length != tokens * N")
    ptrs = (C.c_void_p * len(ws))(*[o.ctypes.data for o in outs])
    nw = None if norm_w is None else _np_ptr(_host_f32(norm_w, "norm_w"))
    ctx.check(lib().lgh_q4_norm_gemv(ctx.handle, len(ws), handles, nw, float(eps), _np_ptr(hidden), ptrs, tokens,
                                     mode))


def ffn_gate_up(w1: Q4Matrix, w3: Q4Matrix, norm_w, eps: float, hidden):
    """The gate/up stage of ffn_residual alone (test hook): returns g, u, h = silu(g) * u and
    h's PerBlock ActQ8 codes / scales as the down projection consumes them."""
    ctx = w1.ctx
    _check_norm_w(norm_w, w1.k)
    hidden = _host_f32(hidden, "hidden")
    _shape_assert(hidden.size == w1.k, "hidden length != dim")
    n = w1.n
    g, u, h = (np.zeros(n, dtype=np.float32) for _ in range(3))
    hq = np.zeros(n, dtype=np.int8)
    hs = np.zeros(n // 32, dtype=np.float32)
    nw = None if norm_w is None else _np_ptr(_host_f32(norm_w, "norm_w"))
    ctx.check(lib().lgh_q4_ffn_gate_up(ctx.handle, w1.handle, w3.handle, nw, float(eps), _np_ptr(hidden),
                                       _np_ptr(g), _np_ptr(u), _np_ptr(h), _np_ptr(hq), _np_ptr(hs)))
    return g, u, h, hq, hs


def q8_apply(m: Q8Matrix, x, tokens: int, out) -> None:
    """q8_apply (crates/llm-engine/src/weights.rs:194-227)."""
    ctx = m.ctx
    if _is_torch(x):
        _shape_assert(x.numel() == tokens * m.k and out.numel() == tokens * m.n, "length mismatch")
        xp, op = _dev_ptr(x, "x"), _dev_ptr(out, "out")
        ctx.dev_call(lambda: ctx.check(lib().lgh_q8_gemv_dev(ctx.handle, m.handle, xp, op, tokens)))
        return
    x = _host_f32(x, "x")
    out = _host_f32(out, "out")
    _shape_assert(x.size == tokens * m.k and out.size == tokens * m.n, "length mismatch")
    ctx.check(lib().lgh_q8_gemv(ctx.handle, m.handle, _np_ptr(x), _np_ptr(out), tokens))


def q8_norm_apply(m: Q8Matrix, norm_w, eps: float, hidden, tokens: int, out) -> None:
    """The final rms_norm then the Q8_0 head (crates/llm-engine/src/lfm2.rs:559-567): per token
    out = W rms_norm(hidden, norm_w, eps) (norm_w None: no norm), the norm in the GEMV's prologue."""
    ctx = m.ctx
    _check_norm_w(norm_w, m.k)
    if _is_torch(hidden):
        _shape_assert(hidden.numel() == tokens * m.k and out.numel() == tokens * m.n, "length mismatch")
        nw = None if norm_w is None else _dev_ptr(norm_w, "norm_w")
        hp, op = _dev_ptr(hidden, "hidden"), _dev_ptr(out, "out")
        ctx.dev_call(lambda: ctx.check(lib().lgh_q8_norm_gemv_dev(ctx.handle, m.handle, nw, float(eps), hp, op,
                                                                  tokens)))
        return
    hidden = _host_f32(hidden, "hidden")
    out = _host_f32(out, "out")
    _shape_assert(hidden.size == tokens * m.k and out.size == tokens * m.n, "length mismatch")
    nw = None if norm_w is None else _np_ptr(_host_f32(norm_w, "norm_w"))
    ctx.check(lib().lgh_q8_norm_gemv(ctx.handle, m.handle, nw, float(eps), _np_ptr(hidden), _np_ptr(out), tokens))


# ---- test hooks ---------------------------------------------------------------------
def q4_block_dots(blocks: np.ndarray, a: np.ndarray, ctx: Context | None = None) -> np.ndarray:
    """Device per-block dots nibble(W) . a (dot_q4_q8_scalar, gemv_q4.rs:959-966)."""
    ctx = ctx or default_context()
    blocks = np.ascontiguousarray(blocks.ravel())
    a = np.ascontiguousarray(a, dtype=np.int8).reshape(-1)
    assert blocks.dtype == BLOCK_Q4 and a.size == blocks.size * 32
    out = np.zeros(blocks.size, dtype=np.int32)
    ctx.check(lib().lgh_q4_block_dots(ctx.handle, _np_ptr(blocks), _np_ptr(a), blocks.size, _np_ptr(out)))
    return out


def q8_block_dots(blocks: np.ndarray, a: np.ndarray, ctx: Context | None = None) -> np.ndarray:
    ctx = ctx or default_context()
    blocks = np.ascontiguousarray(blocks.ravel())
    a = np.ascontiguousarray(a, dtype=np.int8).reshape(-1)
    assert blocks.dtype == BLOCK_Q8_0 and a.size == blocks.size * 32
    out = np.zeros(blocks.size, dtype=np.int32)
    ctx.check(lib().lgh_q8_block_dots(ctx.handle, _np_ptr(blocks), _np_ptr(a), blocks.size, _np_ptr(out)))
    return out


def q4_mfma_block_dots(w: Q4Matrix, qs: np.ndarray, m: int) -> np.ndarray:
    """Per-(token, row, block) integer dots via the GEMM's MFMA operand path."""
    qs = np.ascontiguousarray(qs, dtype=np.int8).reshape(m, w.k)
    out = np.zeros((m, w.n, w.k // 32), dtype=np.int32)
    w.ctx.check(lib().lgh_q4_mfma_block_dots(w.ctx.handle, w.handle, _np_ptr(qs), m, _np_ptr(out)))
    return out
