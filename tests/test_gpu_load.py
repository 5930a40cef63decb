"""Load-time path on the GPU: a safetensors weight decoded to fp32, quantized on the device
(Linear::from_f32, weights.rs:22-48) bit-exactly as the oracle's BlockQ4::quantize, then
applied (Linear::apply, weights.rs:75-88) within the GEMV / GEMM tolerance."""

import numpy as np
import pytest

from llmhost_amd import load, synth

from .conftest import assert_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_linear_from_safetensors(gpu_ctx, oracle, tmp_path, dtype):
    import torch
    from safetensors.torch import save_file

    rows, cols = 96, 256
    w = torch.from_numpy(synth.activations(5, rows, cols) * np.float32(0.05)).to(getattr(torch, dtype))
    path = tmp_path / "w.safetensors"
    save_file({"model.layers.0.feed_forward.w1.weight": w}, str(path))
    t = load.get_tensor(load.load_safetensors_f32(path), "layers.0.feed_forward.w1.weight")
    lin = load.linear_from_tensor(t, ctx=gpu_ctx)
    wf = w.float().numpy()
    blocks = oracle.quantize_q4(wf)
    assert lin.mat.blocks().tobytes() == blocks.tobytes()
    ref_mat = oracle.Q4Matrix(rows, cols, blocks)
    for tokens in (1, 3):
        x = synth.activations(6 + tokens, tokens, cols)
        out = np.zeros(tokens * rows, np.float32)
        lin.apply(x, tokens, out)
        ref = oracle.gemv_q4(ref_mat, x.ravel()) if tokens == 1 else oracle.gemm_q4(ref_mat, x, tokens).ravel()
        assert_close(out, ref, what=f"{dtype} tokens={tokens}")
