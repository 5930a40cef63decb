"""The C-ABI library loads without a GPU and exports every declared symbol.

No compute is called here (this runs on machines without a GPU); the only
calls are ones that never touch a device.
"""

import ctypes as C
import os
import re

import pytest

from llmhost_amd import _ffi


def _declared_functions():
    text = open(_ffi.HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lgh_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = _declared_functions()
    for must in ("lgh_init", "lgh_q4_upload", "lgh_q4_gemv", "lgh_q4_gemv_pair", "lgh_q4_gemm",
                 "lgh_q8_gemv", "lgh_act_quant", "lgh_q4_block_dots"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(_ffi.LIB_PATH)
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_ctypes_signatures_cover_the_header():
    assert set(_declared_functions()) == set(_ffi.SIGNATURES)


def test_version_and_null_handling_without_device():
    lib = _ffi.lib()
    assert b"gfx950" in lib.lgh_version()
    # Calls on a null context fail cleanly instead of crashing.
    assert lib.lgh_sync(None) == _ffi.LGH_ERR_INVALID_ARG
    assert lib.lgh_set_act_quant(None, 0) == _ffi.LGH_ERR_INVALID_ARG
    assert lib.lgh_q4_gemv(None, None, None, None, 0) == _ffi.LGH_ERR_INVALID_ARG
    assert lib.lgh_q4_rows(None) == 0
    lib.lgh_q4_free(None)
    lib.lgh_destroy(None)


def test_init_reports_missing_device_or_wrong_arch():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present; covered by the gpu tests")
    lib = _ffi.lib()
    h = C.c_void_p()
    code = lib.lgh_init(0, C.byref(h))
    assert code in (_ffi.LGH_ERR_NO_DEVICE, _ffi.LGH_ERR_HIP, _ffi.LGH_ERR_ARCH)
    assert not h.value
    assert lib.lgh_last_error(None)


def test_every_gemv_plan_has_a_compiled_kernel():
    """The Q4 and Q8_0 GEMV planners and the ragged (2-64 token) matrix-core planner only choose
    launch shapes the library compiled (a plan without a kernel would fail at launch with
    LGH_ERR_HIP): host-only sweep in the library."""
    assert _ffi.lib().lgh_gemv_plans_uncovered() == 0


def test_cpp_header_compiles_and_matches_the_block_formats(tmp_path):
    """include/llm_gpu_hip.hpp (the C++ host interface) compiles on its own as C++17 with
    warnings as errors, and its block structs have the reference's sizes (18 / 34 bytes)."""
    import subprocess

    src = tmp_path / "t.cpp"
    src.write_text('#include "llm_gpu_hip.hpp"\n'
                   "static_assert(sizeof(llm_gpu_hip::BlockQ4) == 18, \"q4\");\n"
                   "static_assert(sizeof(llm_gpu_hip::BlockQ8_0) == 34, \"q8\");\n"
                   "int main() { return llm_gpu_hip::f16_to_f32(0x3C00) == 1.0f ? 0 : 1; }\n")
    inc = os.path.dirname(_ffi.HEADER_PATH)
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-fsyntax-only", "-I", inc, str(src)],
                   check=True)


def test_rust_ffi_in_integration_doc_declares_every_export():
    """INTEGRATION.md's src/ffi.rs block has one declaration per function of the C header, with the
    same parameter count, so the Rust crate written from it binds the whole boundary."""
    integ = open(os.path.join(os.path.dirname(_ffi.HEADER_PATH), "..", "INTEGRATION.md")).read()
    start = integ.index('extern "C" {')
    block = integ[start:integ.index("\n}\n", start)]
    rust = {}
    for name, params in re.findall(r"pub fn (lgh_\w+)\(([^)]*)\)", block, flags=re.S):
        assert name not in rust, f"{name} declared twice"
        rust[name] = 0 if not params.strip() else params.count(":")
    text = re.sub(r"/\*.*?\*/", "", open(_ffi.HEADER_PATH).read(), flags=re.S)
    header = {}
    for name, params in re.findall(r"\b(lgh_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        params = params.strip()
        header[name] = 0 if params in ("", "void") else params.count(",") + 1
    assert set(rust) == set(header), (sorted(set(header) - set(rust)), sorted(set(rust) - set(header)))
    for name, n in header.items():
        assert rust[name] == n, f"{name}: {rust[name]} Rust parameters, {n} in the header"
