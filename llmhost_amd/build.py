"""Build libllm_gpu_hip.so (gfx950) in-tree with hipcc.

Usage: ``python -m llmhost_amd.build`` (also called by ``__graft_entry__.build()``).
The library is written next to this file so it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libllm_gpu_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ["lgh_api.hip", "lgh_gemv.hip", "lgh_gemm.hip", "lgh_quant.hip", "lgh_ffn.hip", "lgh_probe.hip"]
ARCH = "gfx950"

# Packed FP32 VALU ops are disabled on purpose: every kernel here is written
# against plain fp32 VALU instructions.  MFMA results go to arch VGPRs (not
# AGPRs): the GEMM folds every MFMA result with VALU FMAs, and AGPR results
# would cost a v_accvgpr_read per element.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libllm_gpu_hip.so)")


def build(verbose: bool = False) -> str:
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *HIP_FLAGS, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # The host compiler pass does not know the gfx950 target feature and warns; drop that line.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = [ln for ln in (proc.stdout + proc.stderr).splitlines() if noise not in ln]
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs))
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
