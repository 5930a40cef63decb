"""Load-time path (crates/llm-engine/src/load.rs:120-215): the safetensors decoder against the
safetensors library's own torch loader (which widens BF16 / F16 exactly), the error cases of
tensor_to_f32, and get_tensor's `model.` prefix rule.  CPU only."""

import json
import struct

import numpy as np
import pytest

from llmhost_amd import load
from llmhost_amd.weights import LoadError


def _save(path, tensors):
    from safetensors.torch import save_file

    save_file(tensors, str(path))


def test_decoder_matches_the_safetensors_loader(tmp_path):
    import torch
    from safetensors.torch import load_file

    g = torch.Generator().manual_seed(3)
    src = {
        "model.layers.0.w1.weight": (torch.randn(48, 64, generator=g) * 3).to(torch.bfloat16),
        "layers.0.w2.weight": torch.randn(64, 48, generator=g).to(torch.float16),
        "embed": torch.randn(10, 32, generator=g),
        "scalar": torch.tensor(2.5),
        "empty": torch.zeros(0, 32),
    }
    src["embed"][0, :4] = torch.tensor([float("inf"), -0.0, 1e-40, float("nan")])
    path = tmp_path / "m.safetensors"
    _save(path, src)
    ours = load.load_safetensors_f32(path)
    ref = load_file(str(path))
    assert set(ours) == set(ref)
    for name, t in ref.items():
        want = t.float().numpy().ravel()
        got = ours[name]
        assert got.shape == list(t.shape)
        assert got.data.dtype == np.float32
        assert got.data.view(np.uint32).tobytes() == want.view(np.uint32).tobytes(), name


def test_unsupported_dtype_and_bad_files(tmp_path):
    import torch

    path = tmp_path / "ints.safetensors"
    _save(path, {"ids": torch.arange(8, dtype=torch.int32)})
    with pytest.raises(LoadError, match="unsupported safetensors dtype I32"):
        load.load_safetensors_f32(path)
    with pytest.raises(LoadError, match="not 4-byte aligned"):
        load.tensor_to_f32("F32", b"\x00" * 6)
    with pytest.raises(LoadError, match="bf16 tensor is not 2-byte aligned"):
        load.tensor_to_f32("BF16", b"\x00" * 3)
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes(b"\x05")
    with pytest.raises(LoadError):
        load.load_safetensors_f32(bad)
    # a header that points past the data section
    hdr = json.dumps({"w": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}).encode()
    short = tmp_path / "short.safetensors"
    short.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\x00" * 8)
    with pytest.raises(LoadError, match="invalid offsets"):
        load.load_safetensors_f32(short)
    with pytest.raises(LoadError):
        load.load_safetensors_f32(tmp_path / "missing.safetensors")


def test_get_tensor_model_prefix():
    t = load.TensorF32([1], np.ones(1, np.float32))
    m = {"model.a": t, "b": t}
    assert load.get_tensor(m, "a") is t           # prefix added
    assert load.get_tensor(m, "model.b") is t     # prefix removed
    assert load.get_tensor(m, "model.a") is t
    with pytest.raises(LoadError, match="missing tensor c"):
        load.get_tensor(m, "c")


def test_linear_from_tensor_rejects_non_matrices():
    with pytest.raises(LoadError, match="2-D"):
        load.linear_from_tensor(load.TensorF32([4, 4, 2], np.zeros(32, np.float32)))
