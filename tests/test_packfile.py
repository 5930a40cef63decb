"""The device-image file container on the CPU: header round trip, alignment, and the checks that
turn a damaged file into an error (no device needed: the images here are synthetic bytes)."""

import numpy as np
import pytest

from llmhost_amd import packfile, synth
from llmhost_amd._ffi import LghShapeError


def test_write_and_index_round_trip(tmp_path):
    p = str(tmp_path / "m.lghb")
    a = np.frombuffer(synth.splitmix64(1, 100).tobytes(), dtype=np.uint8)[:777].copy()
    b = np.arange(300, dtype=np.uint8)
    packfile.write_raw(p, {"w.q": ("q4", 64, 96, False, a), "head": ("q8", 10, 32, False, b)})
    tensors, start = packfile.read_index(p)
    assert start % 256 == 0
    assert tensors["w.q"] == {"kind": "q4", "n": 64, "k": 96, "gemm": False, "offset": 0, "bytes": 777}
    assert tensors["head"]["offset"] == 1024 and tensors["head"]["bytes"] == 300
    raw = np.fromfile(p, dtype=np.uint8)
    assert np.array_equal(raw[start:start + 777], a)
    assert np.array_equal(raw[start + 1024:start + 1324], b)


def test_damaged_files_are_rejected(tmp_path):
    p = str(tmp_path / "bad.lghb")
    with open(p, "wb") as f:
        f.write(b"NOPE" + bytes(20))
    with pytest.raises(LghShapeError, match="not a device-image"):
        packfile.read_index(p)
    good = str(tmp_path / "good.lghb")
    packfile.write_raw(good, {"x": ("q4", 1, 32, False, np.zeros(18, np.uint8))})
    data = open(good, "rb").read()
    trunc = str(tmp_path / "trunc.lghb")
    with open(trunc, "wb") as f:
        f.write(data[:-10])
    with pytest.raises(LghShapeError, match="outside the file"):
        packfile.read_index(trunc)


def test_images_of_another_layout_are_rejected(tmp_path):
    """The library copies an image back unchecked, so a file written for another image layout
    (a stale GEMM record format) must not load."""
    lay = packfile.image_layout()
    assert lay & 0xFFFF == 1792  # the GEMM weight record size
    p = str(tmp_path / "old.lghb")
    packfile.write_raw(p, {"x": ("q4", 1, 32, False, np.zeros(18, np.uint8))}, layout=lay + (1 << 16))
    with pytest.raises(LghShapeError, match="layout"):
        packfile.read_index(p)
    ok = str(tmp_path / "ok.lghb")
    packfile.write_raw(ok, {"x": ("q4", 1, 32, False, np.zeros(18, np.uint8))})
    assert packfile.read_index(ok)[0]["x"]["bytes"] == 18
