"""Device images through a file: export -> file -> import gives byte-identical planes (and GEMM
image) and bit-identical results, with no repack on load."""

import numpy as np
import pytest

from llmhost_amd import packfile, q4, synth

pytestmark = pytest.mark.gpu


def test_q4_and_q8_round_trip_through_a_file(gpu_ctx, tmp_path):
    n, k = 640, 2048
    b4 = synth.q4_blocks(5001, n, k)
    b8 = synth.q8_blocks(5002, 300, 1536)
    w = q4.Q4Matrix.from_blocks(n, k, b4, gpu_ctx)
    h = q4.Q8Matrix.from_blocks(300, 1536, b8, gpu_ctx)
    plain, withg = str(tmp_path / "plain.lghb"), str(tmp_path / "gemm.lghb")
    packfile.save(plain, {"w": w, "head": h})
    packfile.save(withg, {"w": w}, with_gemm=True)
    img_plain, img_gemm = packfile.export_image(w), packfile.export_image(w, True)
    assert img_plain.size == n * (k // 32) * 18
    assert np.array_equal(img_gemm[:img_plain.size], img_plain)
    loaded = packfile.load(plain, gpu_ctx)
    loaded_g = packfile.load(withg, gpu_ctx)
    w2, h2, w3 = loaded["w"], loaded["head"], loaded_g["w"]
    # byte-identical planes and image
    assert w2.blocks().tobytes() == b4.tobytes() and h2.blocks().tobytes() == b8.tobytes()
    assert np.array_equal(packfile.export_image(w2), img_plain)
    assert w3.device_bytes() == w.device_bytes()  # the GEMM image came with the file
    assert np.array_equal(packfile.export_image(w3, True), img_gemm)
    assert w2.device_bytes() < w3.device_bytes()  # no image until a GEMM needs it
    # bit-identical results on the GEMV and the GEMM routes
    for m in (1, 130):
        x = synth.activations(5003 + m, m, k)
        ys = [np.zeros((m, n), np.float32) for _ in range(3)]
        for mat, y in zip((w, w2, w3), ys):
            q4.gemm_q4(mat, x, y, m)
        assert np.array_equal(ys[0], ys[1]) and np.array_equal(ys[0], ys[2])
    x8 = synth.normal_f32(5004, 1536)
    a, b = np.zeros(300, np.float32), np.zeros(300, np.float32)
    q4.q8_apply(h, x8, 1, a)
    q4.q8_apply(h2, x8, 1, b)
    assert np.array_equal(a, b)
    with pytest.raises(q4.LghShapeError):
        packfile.import_image("q4", img_plain[:-1], n, k, False, gpu_ctx)
    for m_ in (w, h, w2, h2, w3):
        m_.free()
