"""ctypes declarations for libllm_gpu_hip.so (include/llm_gpu_hip.h).

Loading fails loudly when the library is missing: there is no CPU fallback
for any entry point.
"""

from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libllm_gpu_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "llm_gpu_hip.h")

LGH_OK = 0
LGH_ERR_INVALID_ARG = -1
LGH_ERR_SHAPE = -2
LGH_ERR_HIP = -3
LGH_ERR_ARCH = -4
LGH_ERR_NO_DEVICE = -5
LGH_ERR_OOM = -6
LGH_ERR_CAPTURE = -7

LGH_ASSIGN = 0
LGH_ADD_F64 = 1
LGH_ADD_F32 = 2
LGH_ACT_PER_BLOCK = 0
LGH_ACT_PER_ROW = 1

_P = C.c_void_p
_SZ = C.c_size_t
_I = C.c_int

# name -> (restype, argtypes)
SIGNATURES = {
    "lgh_version": (C.c_char_p, []),
    "lgh_init": (_I, [_I, C.POINTER(_P)]),
    "lgh_destroy": (None, [_P]),
    "lgh_last_error": (C.c_char_p, [_P]),
    "lgh_set_act_quant": (_I, [_P, _I]),
    "lgh_get_act_quant": (_I, [_P]),
    "lgh_set_stream": (_I, [_P, _P]),
    "lgh_get_stream": (_P, [_P]),
    "lgh_sync": (_I, [_P]),
    "lgh_trim": (_I, [_P]),
    "lgh_buffer_alloc": (_I, [_P, _SZ, C.POINTER(_P)]),
    "lgh_buffer_free": (None, [_P, _P]),
    "lgh_buffer_write": (_I, [_P, _P, _P, _SZ]),
    "lgh_buffer_read": (_I, [_P, _P, _P, _SZ]),
    "lgh_q4_upload": (_I, [_P, _P, _SZ, _SZ, C.POINTER(_P)]),
    "lgh_q4_upload_dev": (_I, [_P, _P, _SZ, _SZ, C.POINTER(_P)]),
    "lgh_q4_from_f32": (_I, [_P, _P, _SZ, _SZ, C.POINTER(_P)]),
    "lgh_q4_download": (_I, [_P, _P, _P]),
    "lgh_q4_prepare_gemm": (_I, [_P, _P]),
    "lgh_q4_device_bytes": (_SZ, [_P]),
    "lgh_image_layout": (C.c_uint32, []),
    "lgh_q4_image_bytes": (_SZ, [_P, _I]),
    "lgh_q4_export": (_I, [_P, _P, _I, _P, _SZ]),
    "lgh_q4_import": (_I, [_P, _P, _SZ, _SZ, _SZ, _I, C.POINTER(_P)]),
    "lgh_q8_image_bytes": (_SZ, [_P]),
    "lgh_q8_export": (_I, [_P, _P, _P, _SZ]),
    "lgh_q8_import": (_I, [_P, _P, _SZ, _SZ, _SZ, C.POINTER(_P)]),
    "lgh_q4_free": (None, [_P]),
    "lgh_q4_rows": (_SZ, [_P]),
    "lgh_q4_cols": (_SZ, [_P]),
    "lgh_q8_upload": (_I, [_P, _P, _SZ, _SZ, C.POINTER(_P)]),
    "lgh_q8_from_f32": (_I, [_P, _P, _SZ, _SZ, C.POINTER(_P)]),
    "lgh_q8_download": (_I, [_P, _P, _P]),
    "lgh_q8_free": (None, [_P]),
    "lgh_q8_rows": (_SZ, [_P]),
    "lgh_q8_cols": (_SZ, [_P]),
    "lgh_q4_gemv": (_I, [_P, _P, _P, _P, _I]),
    "lgh_q4_gemv_dev": (_I, [_P, _P, _P, _P, _I]),
    "lgh_q4_gemv_pair": (_I, [_P, _P, _P, _P, _P, _P]),
    "lgh_q4_gemv_pair_dev": (_I, [_P, _P, _P, _P, _P, _P]),
    "lgh_q4_gemm": (_I, [_P, _P, _P, _P, _SZ, _I]),
    "lgh_q4_gemm_dev": (_I, [_P, _P, _P, _P, _SZ, _I]),
    "lgh_q4_gemm_dev_noalloc": (_I, [_P, _P, _P, _P, _SZ, _I]),
    "lgh_probe_empty_dev": (_I, [_P, _I]),
    "lgh_probe_read_outputs": (_SZ, [_SZ, _I]),
    "lgh_probe_read_dev": (_I, [_P, _P, _SZ, _I, _P]),
    "lgh_q8_gemv": (_I, [_P, _P, _P, _P, _SZ]),
    "lgh_q8_gemv_dev": (_I, [_P, _P, _P, _P, _SZ]),
    "lgh_act_quant": (_I, [_P, _P, _SZ, _SZ, _P, _P, _P]),
    "lgh_act_quant_dev": (_I, [_P, _P, _SZ, _SZ, _P, _P, _P]),
    "lgh_q4_gemv_prep": (_I, [_P, _P, _P, _P, _P, _I]),
    "lgh_q4_gemv_prep_dev": (_I, [_P, _P, _P, _P, _P, _I]),
    "lgh_q4_block_dots": (_I, [_P, _P, _P, _SZ, _P]),
    "lgh_q8_block_dots": (_I, [_P, _P, _P, _SZ, _P]),
    "lgh_gemv_plans_uncovered": (_I, []),
    "lgh_q4_mfma_block_dots": (_I, [_P, _P, _P, _SZ, _P]),
    "lgh_rms_norm": (_I, [_P, _P, _P, _SZ, _SZ, C.c_float, _P]),
    "lgh_rms_norm_dev": (_I, [_P, _P, _P, _SZ, _SZ, C.c_float, _P]),
    "lgh_silu_mul": (_I, [_P, _P, _P, _SZ]),
    "lgh_silu_mul_dev": (_I, [_P, _P, _P, _SZ]),
    "lgh_q4_ffn_residual": (_I, [_P, _P, _P, _P, _P, C.c_float, _P, _SZ]),
    "lgh_q4_ffn_residual_dev": (_I, [_P, _P, _P, _P, _P, C.c_float, _P, _SZ]),
    "lgh_q4_ffn_gate_up": (_I, [_P, _P, _P, _P, C.c_float, _P, _P, _P, _P, _P, _P]),
    "lgh_q4_norm_gemv": (_I, [_P, _SZ, _P, _P, C.c_float, _P, _P, _SZ, _I]),
    "lgh_q4_norm_gemv_dev": (_I, [_P, _SZ, _P, _P, C.c_float, _P, _P, _SZ, _I]),
    "lgh_q8_norm_gemv": (_I, [_P, _P, _P, C.c_float, _P, _P, _SZ]),
    "lgh_q8_norm_gemv_dev": (_I, [_P, _P, _P, C.c_float, _P, _P, _SZ]),
}

_lib = None


class LghError(RuntimeError):
    """A negative LGH_ERR_* status from the library."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class LghShapeError(LghError, ValueError):
    """LGH_ERR_SHAPE: the reference would have panicked on an assert."""


def lib() -> C.CDLL:
    """Load the built library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        # One HIP runtime per process: torch ships its own libamdhip64
        # (SONAME libamdhip64.so.7).  Loading torch first lets the dynamic
        # loader satisfy this library's libamdhip64.so.7 with that same copy;
        # loading ours first would make torch bring in a second runtime,
        # which then finds no device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m llmhost_amd.build` "
                "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(code: int, ctx_handle=None) -> None:
    if code == LGH_OK:
        return
    msg = lib().lgh_last_error(ctx_handle).decode(errors="replace")
    if code == LGH_ERR_SHAPE:
        raise LghShapeError(code, msg)
    raise LghError(code, msg)
