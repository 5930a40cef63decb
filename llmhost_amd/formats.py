"""llm-quant block formats as numpy structured dtypes (consumed as-is).

``BlockQ4``   (crates/llm-quant/src/lib.rs:54-58): LE f16 scale + 16 bytes of
two's-complement nibbles; element i sits in the low nibble of qs[i/2] when i
is even, in the high nibble when odd (lib.rs:83-92).  18 bytes.
``BlockQ8_0`` (crates/llm-quant/src/lib.rs:17-21): LE f16 scale + 32 int8.
34 bytes.  Neither Rust struct is #[repr(C)]; this is their natural layout
(a 2-byte f16 then bytes, alignment 2), pinned here by the itemsize asserts
and in C by the sizes in include/llm_gpu_hip.h.
"""

from __future__ import annotations

import numpy as np

BLOCK_SIZE = 32  # crates/llm-quant/src/lib.rs:12

BLOCK_Q4 = np.dtype([("scale", "<u2"), ("qs", "u1", (16,))])
BLOCK_Q8_0 = np.dtype([("scale", "<u2"), ("qs", "i1", (32,))])
assert BLOCK_Q4.itemsize == 18
assert BLOCK_Q8_0.itemsize == 34


def q4_nibbles(blocks: np.ndarray) -> np.ndarray:
    """Signed nibble values (-8..7) of BlockQ4 blocks, shape [..., 32]."""
    qs = blocks["qs"].astype(np.uint8)
    lo = (qs & 0x0F).astype(np.int8)
    hi = (qs >> 4).astype(np.int8)
    out = np.empty(qs.shape[:-1] + (32,), dtype=np.int8)
    out[..., 0::2] = ((lo ^ 8) - 8)
    out[..., 1::2] = ((hi ^ 8) - 8)
    return out


def q4_from_nibbles(nibbles: np.ndarray, scale_bits: np.ndarray) -> np.ndarray:
    """Pack signed nibbles [..., 32] (-8..7) and f16 scale bits into BlockQ4."""
    nib = (np.asarray(nibbles).astype(np.int16) & 0xF).astype(np.uint8)
    out = np.zeros(nib.shape[:-1], dtype=BLOCK_Q4)
    out["qs"] = nib[..., 0::2] | (nib[..., 1::2] << 4)
    out["scale"] = scale_bits
    return out
