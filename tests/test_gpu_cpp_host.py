"""The C++ host interface (include/llm_gpu_hip.hpp) on the GPU: runs tests/cpp/host_api_test,
the reference's own unit tests for this path (llm-quant lib.rs:143-222, llm-cpu gemv_q4.rs
tests, the llm-engine seam, the llm-core Backend / Block traits) written against the C++ mirror
(see tests/cpp/host_api_test.cpp).  The binary is built by __graft_entry__.build()."""

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
EXE = os.path.join(HERE, "cpp", "host_api_test")


def test_cpp_host_interface():
    assert os.path.exists(EXE), f"{EXE} is not built: run __graft_entry__.build()"
    proc = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    print(proc.stderr)
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-2000:]
    assert "PASSED: 0 failed" in proc.stdout
    started, passed = proc.stdout.count("[test] "), proc.stdout.count("[ok] ")
    assert started == passed >= 15, proc.stdout
