"""Load-time path: safetensors -> fp32 -> device-quantized matrices.

Restates ``load_safetensors_f32`` / ``tensor_to_f32`` / ``get_tensor``
(crates/llm-engine/src/load.rs:120-215): every tensor of a ``.safetensors``
file decoded to fp32 (F32, BF16 and F16; any other dtype is a ``LoadError``),
looked up by name or with the ``model.`` prefix added or removed.  The file is
memory-mapped and parsed directly (8-byte little-endian header length, JSON
header, data section), so BF16 needs no framework.  ``linear_from_tensor``
then quantizes on the device (``Linear::from_f32``, weights.rs:22-48).
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass

import numpy as np

from .weights import Linear, LoadError, WeightFormat

_DTYPE_BYTES = {"F64": 8, "F32": 4, "F16": 2, "BF16": 2, "I64": 8, "I32": 4, "I16": 2, "I8": 1, "U8": 1,
                "BOOL": 1, "U16": 2, "U32": 4, "U64": 8, "F8_E4M3": 1, "F8_E5M2": 1}


@dataclass
class TensorF32:
    """TensorF32 (load.rs:45-48): shape and fp32 data."""

    shape: list
    data: np.ndarray


def tensor_to_f32(dtype: str, raw) -> np.ndarray:
    """tensor_to_f32 (load.rs:141-191)."""
    raw = memoryview(raw).cast("B")
    if dtype == "F32":
        if len(raw) % 4:
            raise LoadError("f32 tensor is not 4-byte aligned")
        return np.frombuffer(raw, dtype="<f4").astype(np.float32)
    if dtype == "BF16":
        if len(raw) % 2:
            raise LoadError("bf16 tensor is not 2-byte aligned")
        bits = np.frombuffer(raw, dtype="<u2").astype(np.uint32) << 16
        return bits.view(np.float32)
    if dtype == "F16":
        if len(raw) % 2:
            raise LoadError("f16 tensor is not 2-byte aligned")
        return np.frombuffer(raw, dtype="<f2").astype(np.float32)  # exact: every f16 is an f32
    raise LoadError(f"unsupported safetensors dtype {dtype}")


def _header(mm: np.ndarray, path: str) -> tuple[dict, int]:
    if mm.size < 8:
        raise LoadError(f"{path}: not a safetensors file (shorter than its header length)")
    n = int(np.frombuffer(mm[:8].tobytes(), dtype="<u8")[0])
    if n > mm.size - 8:
        raise LoadError(f"{path}: header length {n} exceeds the file")
    try:
        header = json.loads(mm[8:8 + n].tobytes().decode("utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise LoadError(f"{path}: invalid safetensors header ({e})") from None
    if not isinstance(header, dict):
        raise LoadError(f"{path}: invalid safetensors header")
    return header, 8 + n


def load_safetensors_f32(path) -> dict[str, TensorF32]:
    """load_safetensors_f32 (load.rs:120-139): every tensor of the file as fp32."""
    path = os.fspath(path)
    try:
        mm = np.memmap(path, dtype=np.uint8, mode="r")
    except (OSError, ValueError) as e:
        raise LoadError(str(e)) from None
    header, base = _header(mm, path)
    out: dict[str, TensorF32] = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        try:
            dtype, shape, (b, e) = info["dtype"], list(info["shape"]), info["data_offsets"]
        except (KeyError, TypeError, ValueError):
            raise LoadError(f"{path}: invalid header entry for {name}") from None
        count = int(np.prod(shape, dtype=np.int64)) if shape else 1
        if not (0 <= b <= e <= mm.size - base) or (dtype in _DTYPE_BYTES and e - b != count * _DTYPE_BYTES[dtype]):
            raise LoadError(f"{path}: tensor {name} has invalid offsets [{b}, {e})")
        out[name] = TensorF32(shape, tensor_to_f32(dtype, mm[base + b:base + e]))
    return out


def get_tensor(tensors: dict[str, TensorF32], name: str) -> TensorF32:
    """get_tensor (load.rs:200-215): `name`, else with the `model.` prefix removed or added."""
    if name in tensors:
        return tensors[name]
    alt = name[len("model."):] if name.startswith("model.") else f"model.{name}"
    if alt in tensors:
        return tensors[alt]
    raise LoadError(f"missing tensor {name}")


def linear_from_tensor(t: TensorF32, fmt: str = WeightFormat.Q4_32, ctx=None) -> Linear:
    """A [rows, cols] weight tensor quantized on the device (Linear::from_f32, weights.rs:22-48)."""
    if len(t.shape) != 2:
        raise LoadError(f"linear weight must be 2-D, got shape {t.shape}")
    rows, cols = t.shape
    return Linear.from_f32(t.data, rows, cols, fmt, ctx)
