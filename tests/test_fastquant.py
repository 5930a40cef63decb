"""Exhaustive CPU proof of the device quantizer's fast exact arithmetic.

tests/fastquant_check.c checks, over every relevant float, that the three
shortcuts used by act_quant_group8 (llmhost_amd/csrc/lgh_device.h) are
exactly the IEEE operations llm-cpu performs (crates/llm-cpu/src/gemv_q4.rs:
83-88): amax / 127, 1 / scale, and round-half-away-from-zero of v * inv.
The GPU parity tests then pin the device results bit-exactly.
"""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc is required")
def test_fast_divisions_and_rounding_are_exact(tmp_path):
    exe = tmp_path / "fastquant_check"
    subprocess.run(["gcc", "-O2", "-mfma", "-fopenmp", "-ffp-contract=off",
                    os.path.join(HERE, "fastquant_check.c"), "-o", str(exe), "-lm"], check=True)
    env = dict(os.environ)
    env.setdefault("OMP_NUM_THREADS", str(min(16, len(os.sched_getaffinity(0)))))
    out = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=600)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout + out.stderr
