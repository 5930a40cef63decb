"""llmhost_amd: MI355X (gfx950) block-quantized matmul for llmhost.

A from-scratch HIP implementation of llmhost's Q4_32 / Q8_0 matmul hot path
(fused-dequant GEMV for decode, int8-MFMA GEMM for prefill) behind a C ABI
(include/llm_gpu_hip.h, libllm_gpu_hip.so), with a host-side mirror of the
reference interface:

* ``llmhost_amd.q4``      -- llm-cpu's gemv_q4 / gemm_q4 / ActQ8 / Q4Matrix API;
* ``llmhost_amd.weights`` -- llm-engine's Linear / apply_pair / OutputHead seam;
* ``llmhost_amd.formats`` -- llm-quant's BlockQ4 / BlockQ8_0 byte layouts;
* ``llmhost_amd.synth``   -- seeded synthetic operands for tests and benchmarks.
"""

from .formats import BLOCK_Q4, BLOCK_Q8_0, BLOCK_SIZE  # noqa: F401

__version__ = "0.1.0"


def library_path() -> str:
    from ._ffi import LIB_PATH

    return LIB_PATH
