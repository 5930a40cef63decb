"""A file of device-packed matrices: loading one is a read and one host-to-device copy per matrix,
with no quantization and no repack kernel.

Layout (little-endian):  b"LGHB"  u32 version  u64 header_len  header (UTF-8 JSON)  data.
The header holds "layout" (``lgh_image_layout()`` of the library that wrote the images) and maps
each name to {"kind": "q4" | "q8", "n", "k", "gemm": bool, "offset", "bytes"}; offsets are from
the start of the data section and 256-byte aligned.  A tensor's bytes are the library's device
image of the matrix (``lgh_q4_export`` / ``lgh_q8_export``): the nibble (or code) plane, the f16
scale plane and, for Q4 with "gemm", the GEMM operand image.  The library copies an image back
without checking it, so a file whose layout differs from the loading library's is rejected.

The reference loads safetensors and quantizes at load (crates/llm-engine/src/load.rs:120-191,
Q4Matrix::from_blocks repacking every load, crates/llm-cpu/src/gemv_q4.rs:128-149) and plans a
pre-packed ``.lfmb`` container without a layout yet (ARCHITECTURE.md:101); this is that
pre-packed form for the device layout.
"""

from __future__ import annotations

import ctypes as C
import json
import struct

import numpy as np

from . import q4 as _q4
from ._ffi import LghShapeError, LGH_ERR_SHAPE, lib

MAGIC = b"LGHB"
VERSION = 2
ALIGN = 256


def image_layout() -> int:
    """The device image layout of the loaded library (``lgh_image_layout``)."""
    return int(lib().lgh_image_layout())


def _align(v: int) -> int:
    return (v + ALIGN - 1) // ALIGN * ALIGN


def export_image(mat, with_gemm: bool = False) -> np.ndarray:
    """The device image of a Q4Matrix / Q8Matrix as a uint8 host array."""
    ctx = mat.ctx
    if isinstance(mat, _q4.Q4Matrix):
        nbytes = lib().lgh_q4_image_bytes(mat.handle, int(with_gemm))
        out = np.empty(nbytes, dtype=np.uint8)
        ctx.check(lib().lgh_q4_export(ctx.handle, mat.handle, int(with_gemm), out.ctypes.data_as(C.c_void_p), nbytes))
        return out
    nbytes = lib().lgh_q8_image_bytes(mat.handle)
    out = np.empty(nbytes, dtype=np.uint8)
    ctx.check(lib().lgh_q8_export(ctx.handle, mat.handle, out.ctypes.data_as(C.c_void_p), nbytes))
    return out


def import_image(kind: str, image: np.ndarray, n: int, k: int, with_gemm: bool = False,
                 ctx: _q4.Context | None = None):
    """A Q4Matrix / Q8Matrix from a device image (one host-to-device copy per plane)."""
    ctx = ctx or _q4.default_context()
    image = np.ascontiguousarray(image, dtype=np.uint8)
    h = C.c_void_p()
    ptr = image.ctypes.data_as(C.c_void_p)
    if kind == "q4":
        ctx.check(lib().lgh_q4_import(ctx.handle, ptr, image.size, n, k, int(with_gemm), C.byref(h)))
        return _q4.Q4Matrix(h, n, k, ctx)
    if kind == "q8":
        ctx.check(lib().lgh_q8_import(ctx.handle, ptr, image.size, n, k, C.byref(h)))
        return _q4.Q8Matrix(h, n, k, ctx)
    raise ValueError(f"unknown matrix kind {kind!r}")


def write_raw(path: str, entries: dict, layout: int | None = None) -> None:
    """Write already-exported images: entries[name] = (kind, n, k, gemm, uint8 image), made by a
    library whose ``lgh_image_layout()`` is ``layout`` (default: the loaded library's)."""
    layout = image_layout() if layout is None else int(layout)
    header, off = {}, 0
    for name, (kind, n, k, gemm, img) in entries.items():
        header[name] = {"kind": kind, "n": int(n), "k": int(k), "gemm": bool(gemm), "offset": off,
                        "bytes": int(img.size)}
        off = _align(off + img.size)
    hj = json.dumps({"format": "lghb", "version": VERSION, "layout": layout, "tensors": header},
                    sort_keys=True).encode()
    pre = MAGIC + struct.pack("<IQ", VERSION, len(hj)) + hj
    data_start = _align(len(pre))
    with open(path, "wb") as f:
        f.write(pre)
        f.write(b"\0" * (data_start - len(pre)))
        pos = 0
        for name, (_, _, _, _, img) in entries.items():
            f.write(b"\0" * (header[name]["offset"] - pos))
            f.write(np.ascontiguousarray(img, dtype=np.uint8).tobytes())
            pos = header[name]["offset"] + img.size


def read_index(path: str):
    """(header dict of tensors, data start offset), checking the magic, version and bounds."""
    with open(path, "rb") as f:
        pre = f.read(16)
        if len(pre) < 16 or pre[:4] != MAGIC:
            raise LghShapeError(LGH_ERR_SHAPE, f"{path}: not a device-image file")
        version, hlen = struct.unpack("<IQ", pre[4:])
        if version != VERSION:
            raise LghShapeError(LGH_ERR_SHAPE, f"{path}: version {version}, expected {VERSION}")
        hj = f.read(hlen)
        f.seek(0, 2)
        size = f.tell()
    if len(hj) != hlen:
        raise LghShapeError(LGH_ERR_SHAPE, f"{path}: truncated header")
    meta = json.loads(hj)
    if meta.get("layout") != image_layout():
        raise LghShapeError(LGH_ERR_SHAPE, f"{path}: images of layout {meta.get('layout')!r}, this "
                            f"library reads layout {image_layout()}; export the matrices again")
    start = _align(16 + hlen)
    for name, t in meta["tensors"].items():
        if t["offset"] % ALIGN or start + t["offset"] + t["bytes"] > size:
            raise LghShapeError(LGH_ERR_SHAPE, f"{path}: tensor {name} lies outside the file")
    return meta["tensors"], start


def save(path: str, mats: dict, with_gemm: bool = False) -> None:
    """Write {name: Q4Matrix | Q8Matrix}; with_gemm stores each Q4 matrix's GEMM image as well."""
    entries = {}
    for name, m in mats.items():
        kind = "q4" if isinstance(m, _q4.Q4Matrix) else "q8"
        g = with_gemm and kind == "q4"
        entries[name] = (kind, m.n, m.k, g, export_image(m, g))
    write_raw(path, entries)


def load(path: str, ctx: _q4.Context | None = None) -> dict:
    """{name: Q4Matrix | Q8Matrix} from a device-image file (memory-mapped, one copy per matrix)."""
    tensors, start = read_index(path)
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    out = {}
    for name, t in tensors.items():
        img = np.asarray(mm[start + t["offset"]:start + t["offset"] + t["bytes"]])
        out[name] = import_image(t["kind"], img, t["n"], t["k"], t["gemm"], ctx)
    del mm
    return out
