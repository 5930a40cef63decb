"""Host-side argument checks of the Python mirror that run before any device call (CPU only).

The reference asserts on these (crates/llm-cpu/src/ops.rs:9-11 for the norm weight length);
the mirror raises LghShapeError before the library could read past a short buffer.
"""

import types

import numpy as np
import pytest

from llmhost_amd import q4


def _mat(n, k):
    return types.SimpleNamespace(n=n, k=k, ctx=None, handle=None)


def test_norm_gemv_rejects_short_norm_weight():
    with pytest.raises(q4.LghShapeError, match="norm weight"):
        q4.norm_gemv([_mat(64, 128)], np.ones(127, np.float32), 1e-5, np.zeros(128, np.float32),
                     [np.zeros(64, np.float32)])


def test_ffn_residual_rejects_short_norm_weight():
    w1, w3, w2 = _mat(256, 128), _mat(256, 128), _mat(128, 256)
    with pytest.raises(q4.LghShapeError, match="norm weight"):
        q4.ffn_residual(w1, w3, w2, np.ones(64, np.float32), 1e-5, np.zeros(128, np.float32))


def test_ffn_gate_up_rejects_short_norm_weight():
    with pytest.raises(q4.LghShapeError, match="norm weight"):
        q4.ffn_gate_up(_mat(256, 128), _mat(256, 128), np.ones(96, np.float32), 1e-5, np.zeros(128, np.float32))


def test_q8_norm_apply_rejects_short_norm_weight():
    with pytest.raises(q4.LghShapeError, match="norm weight"):
        q4.q8_norm_apply(_mat(64, 128), np.ones(32, np.float32), 1e-5, np.zeros(128, np.float32), 1,
                         np.zeros(64, np.float32))


def test_norm_weight_of_the_right_length_passes_the_check():
    q4._check_norm_w(np.ones(128, np.float32), 128)
    q4._check_norm_w(None, 128)
    with pytest.raises(q4.LghShapeError):
        q4._check_norm_w(np.ones(129, np.float32), 128)
