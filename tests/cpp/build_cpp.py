"""Build tests/cpp/host_api_test (the C++ host-interface tests) against the in-tree library.

Called by ``__graft_entry__.build()`` after the library is built; g++ only (the test is host
code: it reaches the GPU through libllm_gpu_hip.so).
"""

from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
SRC = os.path.join(HERE, "host_api_test.cpp")
EXE = os.path.join(HERE, "host_api_test")


def build() -> str:
    lib_dir = os.path.join(ROOT, "llmhost_amd")
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-ffp-contract=off",
           "-I", os.path.join(ROOT, "include"), SRC, "-o", EXE + ".tmp",
           "-L", lib_dir, "-lllm_gpu_hip", "-Wl,-rpath,$ORIGIN/../../llmhost_amd"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("g++ failed:\n" + proc.stdout + proc.stderr)
    os.replace(EXE + ".tmp", EXE)
    return EXE


if __name__ == "__main__":
    print(build())
