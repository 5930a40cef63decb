"""CPU oracle for llmhost's Q4_32 / Q8_0 matmul path (TEST INFRASTRUCTURE).

ctypes binding of ``oracle/liboracle.so``, a C restatement of
``crates/llm-quant/src/lib.rs``, ``crates/llm-cpu/src/gemv_q4.rs`` and the
Q8_0 head GEMV in ``crates/llm-engine/src/weights.rs:194-227``.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package: as the reference the GPU path is compared
against, and as the timed CPU baseline.  The product package ``llmhost_amd``
never imports it.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

# llm-quant/src/lib.rs:17-21, 54-58 in their natural (packed, align-2) layout.
BLOCK_Q4 = np.dtype([("scale", "<u2"), ("qs", "u1", (16,))])
BLOCK_Q8 = np.dtype([("scale", "<u2"), ("qs", "i1", (32,))])
assert BLOCK_Q4.itemsize == 18 and BLOCK_Q8.itemsize == 34

KERNEL_DETECT, KERNEL_SCALAR, KERNEL_AVX2, KERNEL_VNNI = -1, 0, 1, 2
KERNEL_AMX = 3  # GEMM only (m >= 16, no add): llm-cpu/src/amx.rs

_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (gcc only)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "liboracle.so"],
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        P = C.c_void_p
        sz = C.c_size_t
        i = C.c_int
        L.oq_f16_to_f32.argtypes, L.oq_f16_to_f32.restype = [C.c_uint16], C.c_float
        L.oq_f32_to_f16.argtypes, L.oq_f32_to_f16.restype = [C.c_float], C.c_uint16
        for name in ("oq_q8_quantize", "oq_q4_quantize"):
            getattr(L, name).argtypes = [P, P]
        L.oq_q4_nibble.argtypes, L.oq_q4_nibble.restype = [P, i], C.c_int8
        L.oq_q4_dequantize.argtypes = [P, P]
        L.oq_q8_dequantize.argtypes = [P, P]
        L.oq_quantize_q4.argtypes, L.oq_quantize_q4.restype = [P, sz, P], i
        L.oq_quantize_q8_0.argtypes, L.oq_quantize_q8_0.restype = [P, sz, P], i
        L.oq_act_quantize.argtypes, L.oq_act_quantize.restype = [P, sz, sz, i, P, P, P], i
        L.oq_dot_q4_q8.argtypes, L.oq_dot_q4_q8.restype = [P, P], C.c_int32
        L.oq_dot_q4_q8_offset.argtypes, L.oq_dot_q4_q8_offset.restype = [P, P, C.c_int32], C.c_int32
        L.oq_dot_q8_q8.argtypes, L.oq_dot_q8_q8.restype = [P, P], C.c_int32
        L.oq_q4_from_blocks.argtypes, L.oq_q4_from_blocks.restype = [sz, sz, P], P
        L.oq_q4_free.argtypes = [P]
        L.oq_detect_kernel.restype = i
        L.oq_gemv_q4.argtypes = [P, P, P, i, i, i, i]
        L.oq_gemv_q4_prep.argtypes = [P, P, P, P, i, i, i]
        L.oq_gemv_q4_pair.argtypes = [P, P, P, P, P, i, i, i]
        L.oq_gemm_q4.argtypes = [P, P, P, sz, i, i, i, i]
        L.oq_q8_apply.argtypes = [P, sz, sz, P, sz, P, i]
        L.oq_rms_norm.argtypes = [P, P, sz, sz, C.c_float, P]
        L.oq_silu_mul.argtypes = [P, P, sz]
        L.oq_ffn_residual.argtypes = [P, P, P, P, C.c_float, P, sz, i, i, i]
        L.oq_thread_range.argtypes = [sz, sz, sz, C.POINTER(sz), C.POINTER(sz)]
        L.oq_cpu_has.argtypes, L.oq_cpu_has.restype = [C.c_char_p], i
        L.oq_amx_ready.restype = i
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


# ---- f16 ---------------------------------------------------------------
def f16_to_f32(bits: int) -> float:
    return lib().oq_f16_to_f32(int(bits))


def f32_to_f16(v: float) -> int:
    return int(lib().oq_f32_to_f16(float(np.float32(v))))


# ---- llm-quant -----------------------------------------------------------
def quantize_q4(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(x.size // 32, dtype=BLOCK_Q4)
    if lib().oq_quantize_q4(_p(x), x.size, _p(out)) != 0:
        raise ValueError("Q4 input length must be a multiple of 32")
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(x.size // 32, dtype=BLOCK_Q8)
    if lib().oq_quantize_q8_0(_p(x), x.size, _p(out)) != 0:
        raise ValueError("Q8_0 input length must be a multiple of 32")
    return out


def q4_nibble(block: np.ndarray, i: int) -> int:
    b = np.ascontiguousarray(block.reshape(1))
    return int(lib().oq_q4_nibble(_p(b), i))


def dequantize_q4(blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks.ravel())
    out = np.zeros(blocks.size * 32, dtype=np.float32)
    for b in range(blocks.size):
        lib().oq_q4_dequantize(_p(blocks[b:b + 1]), C.c_void_p(out.ctypes.data + 128 * b))
    return out


def dequantize_q8_0(blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks.ravel())
    out = np.zeros(blocks.size * 32, dtype=np.float32)
    for b in range(blocks.size):
        lib().oq_q8_dequantize(_p(blocks[b:b + 1]), C.c_void_p(out.ctypes.data + 128 * b))
    return out


# ---- activation quant ------------------------------------------------------
def act_quantize(x: np.ndarray, per_row: bool = False):
    """ActQ8 quantization of x[m, k] (or x[k]); returns (qs, scales, sums)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    m, k = x2.shape
    qs = np.zeros((m, k), dtype=np.int8)
    sc = np.zeros((m, k // 32), dtype=np.float32)
    su = np.zeros((m, k // 32), dtype=np.int32)
    if lib().oq_act_quantize(_p(x2), m, k, int(per_row), _p(qs), _p(sc), _p(su)) != 0:
        raise ValueError(f"activation length {k} is not a multiple of 32")
    shp = x.shape
    return qs.reshape(shp), sc.reshape(shp[:-1] + (k // 32,)), su.reshape(shp[:-1] + (k // 32,))


def dot_q4_q8(block: np.ndarray, a: np.ndarray) -> int:
    b = np.ascontiguousarray(block.reshape(1))
    a = np.ascontiguousarray(a, dtype=np.int8)
    return int(lib().oq_dot_q4_q8(_p(b), _p(a)))


def dot_q4_q8_offset(block: np.ndarray, a: np.ndarray, a_sum: int) -> int:
    b = np.ascontiguousarray(block.reshape(1))
    a = np.ascontiguousarray(a, dtype=np.int8)
    return int(lib().oq_dot_q4_q8_offset(_p(b), _p(a), int(a_sum)))


def dot_q8_q8(block: np.ndarray, a: np.ndarray) -> int:
    b = np.ascontiguousarray(block.reshape(1))
    a = np.ascontiguousarray(a, dtype=np.int8)
    return int(lib().oq_dot_q8_q8(_p(b), _p(a)))


# ---- packed matrix + llm-cpu entry points ----------------------------------
class Q4Matrix:
    """Q4Matrix::from_blocks (gemv_q4.rs:128-149), packed 16-row CPU tiles."""

    def __init__(self, n: int, k: int, blocks: np.ndarray):
        blocks = np.ascontiguousarray(blocks.ravel())
        assert blocks.dtype == BLOCK_Q4 and blocks.size == n * (k // 32)
        self.n, self.k = n, k
        self._blocks = blocks
        self._h = lib().oq_q4_from_blocks(n, k, _p(blocks))
        if not self._h:
            raise ValueError(f"K={k} is not a multiple of 32")

    @classmethod
    def from_f32(cls, w: np.ndarray, n: int, k: int) -> "Q4Matrix":
        return cls(n, k, quantize_q4(w))

    @property
    def handle(self):
        return C.c_void_p(self._h)

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.oq_q4_free(C.c_void_p(self._h))
            self._h = None


def gemv_q4(w: Q4Matrix, x, out=None, add=False, per_row=False, kernel=KERNEL_DETECT, threads=1):
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size == w.k
    if out is None:
        out = np.zeros(w.n, dtype=np.float32)
    lib().oq_gemv_q4(w.handle, _p(x), _p(out), int(add), int(per_row), kernel, threads)
    return out


def gemv_q4_prep(w: Q4Matrix, qs, scales, out=None, add=False, kernel=KERNEL_DETECT, threads=1):
    qs = np.ascontiguousarray(qs, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    if out is None:
        out = np.zeros(w.n, dtype=np.float32)
    lib().oq_gemv_q4_prep(w.handle, _p(qs), _p(scales), _p(out), int(add), kernel, threads)
    return out


def gemv_q4_pair(wg: Q4Matrix, wu: Q4Matrix, x, per_row=False, kernel=KERNEL_DETECT, threads=1):
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert wg.k == wu.k == x.size and wg.n == wu.n
    og = np.zeros(wg.n, dtype=np.float32)
    ou = np.zeros(wu.n, dtype=np.float32)
    lib().oq_gemv_q4_pair(wg.handle, wu.handle, _p(x), _p(og), _p(ou), int(per_row), kernel, threads)
    return og, ou


def gemm_q4(w: Q4Matrix, x, m: int, out=None, add=False, per_row=False, kernel=KERNEL_DETECT,
            threads=1):
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size == m * w.k
    if out is None:
        out = np.zeros((m, w.n), dtype=np.float32)
    lib().oq_gemm_q4(w.handle, _p(x), _p(out), m, int(add), int(per_row), kernel, threads)
    return out


def q8_apply(blocks: np.ndarray, n: int, k: int, x, tokens: int = 1, threads=1):
    blocks = np.ascontiguousarray(blocks.ravel())
    assert blocks.dtype == BLOCK_Q8 and blocks.size == n * (k // 32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size == tokens * k
    out = np.zeros((tokens, n) if tokens > 1 else (n,), dtype=np.float32)
    lib().oq_q8_apply(_p(blocks), n, k, _p(x), tokens, _p(out), threads)
    return out


def rms_norm(x, weight, eps: float):
    """ops.rs:8-23 over the rows of x (row length = weight.size)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    weight = np.ascontiguousarray(weight, dtype=np.float32)
    assert x.size % weight.size == 0
    out = np.empty_like(x)
    lib().oq_rms_norm(_p(x), _p(weight), weight.size, x.size // weight.size, eps, _p(out))
    return out


def silu_mul(g, u):
    """silu(g) * u (ops.rs:27-36, lfm2.rs:902-905), f32."""
    out = np.array(g, dtype=np.float32, copy=True)
    u = np.ascontiguousarray(u, dtype=np.float32)
    assert out.size == u.size
    lib().oq_silu_mul(_p(out), _p(u), out.size)
    return out


def ffn_residual(w1: "Q4Matrix", w3: "Q4Matrix", w2: "Q4Matrix", norm_w, eps: float, hidden, tokens=1,
                 per_row=False, kernel=KERNEL_DETECT, threads=1):
    """Lfm2::ffn_residual / ffn_residual_in (lfm2.rs:861-911); returns the new hidden."""
    out = np.array(hidden, dtype=np.float32, copy=True)
    assert out.size == tokens * w1.k and w1.k == w3.k == w2.n and w1.n == w3.n == w2.k
    nw = None if norm_w is None else np.ascontiguousarray(norm_w, dtype=np.float32)
    lib().oq_ffn_residual(w1.handle, w3.handle, w2.handle, None if nw is None else _p(nw), eps, _p(out),
                          tokens, int(per_row), kernel, threads)
    return out


def detect_kernel() -> int:
    return lib().oq_detect_kernel()


def kernel_name(k: int) -> str:
    return {KERNEL_SCALAR: "scalar", KERNEL_AVX2: "avx2", KERNEL_VNNI: "vnni512", KERNEL_AMX: "amx-int8"}[k]


def amx_ready() -> bool:
    """amx_ready (llm-cpu/src/amx.rs:29-66): the CPU has AMX-TILE and AMX-INT8 and the process
    may use tile data.  gemm_q4 with the detected kernel then takes the AMX tiles for m >= 16
    without add (gemv_q4.rs:711)."""
    return bool(lib().oq_amx_ready())


def thread_range(tid: int, nthreads: int, n: int):
    s, e = C.c_size_t(), C.c_size_t()
    lib().oq_thread_range(tid, nthreads, n, C.byref(s), C.byref(e))
    return s.value, e.value


def cpu_has(feature: str) -> bool:
    return bool(lib().oq_cpu_has(feature.encode()))
