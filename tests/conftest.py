import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


# Output tolerance of the north-star gate: |gpu - cpu| <= 1e-4 + 1e-5 * |cpu|.
ATOL = 1e-4
RTOL = 1e-5


def assert_close(got, ref, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.flatnonzero(bad.ravel())[0]
        raise AssertionError(
            f"{what}: {bad.sum()} / {bad.size} elements out of tolerance; first at flat {i}: "
            f"got {got.ravel()[i]!r} ref {ref.ravel()[i]!r} (max err {err.max():.3e})")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.lib()
    return o


@pytest.fixture(scope="session")
def gpu_ctx():
    # No skip: a gpu-marked test that cannot open the device must fail loudly.
    from llmhost_amd import q4

    return q4.default_context()
