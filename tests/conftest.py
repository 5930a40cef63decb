import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


# Output tolerance against llm-cpu (only summation order differs): |gpu - cpu| <= 1e-4 + 1e-5 * |cpu|.
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


def code_flip_bound(blocks, n, k, q_ref, s_ref, q_got, s_got):
    """Upper bound, per output row, on |W (q_got * s_got) - W (q_ref * s_ref)| in exact arithmetic
    for a Q4 matrix W (BlockQ4 [n, k/32]) applied to two ActQ8 quantizations of (nearly) the same
    vector: q codes [k], s block scales [k/32].  Per block kb with dots D = sum w q:
        |s' D' - s D| <= |s' - s| sum |w| |q'| + s sum |w| |q' - q|,
    times the block's weight scale.  Zero when the codes and scales agree; each flipped code adds
    |nibble| * sw * sa.  Also returns the number of codes and of block scales that differ."""
    from llmhost_amd import formats

    bpr = k // 32
    nib = np.abs(formats.q4_nibbles(blocks.reshape(n, bpr)).astype(np.int64))  # [n, bpr, 32]
    sw = blocks.reshape(n, bpr)["scale"].view(np.float16).astype(np.float64)    # [n, bpr]
    q_ref = np.asarray(q_ref, np.int64).reshape(bpr, 32)
    q_got = np.asarray(q_got, np.int64).reshape(bpr, 32)
    s_ref = np.asarray(s_ref, np.float64).reshape(bpr)
    s_got = np.asarray(s_got, np.float64).reshape(bpr)
    a = np.einsum("ibj,bj->ib", nib, np.abs(q_got))             # sum |w| |q'| per row and block
    b = np.einsum("ibj,bj->ib", nib, np.abs(q_got - q_ref))     # sum |w| |q' - q|
    bound = (sw * (np.abs(s_got - s_ref)[None, :] * a + s_ref[None, :] * b)).sum(axis=1)
    flips = int(np.count_nonzero(q_got != q_ref))
    scale_diffs = int(np.count_nonzero(s_got != s_ref))
    return bound, flips, scale_diffs


def assert_close_with_flips(got, ref, bound, what=""):
    """The gate tolerance plus a per-element allowance (e.g. code_flip_bound's)."""
    got = np.asarray(got, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    bound = np.asarray(bound, dtype=np.float64).ravel()
    err = np.abs(got - ref)
    lim = ATOL + RTOL * np.abs(ref) + bound * (1 + 1e-6)
    bad = err > lim
    if bad.any():
        i = np.flatnonzero(bad)[0]
        raise AssertionError(f"{what}: {bad.sum()} / {bad.size} out of tolerance; first at {i}: got {got[i]!r} "
                             f"ref {ref[i]!r} allowance {bound[i]:.3e}")


def q8_exact_terms(blocks, n, k, qs, sa):
    """q8_apply's value in exact arithmetic for BlockQ8_0 [n, k/32] on ActQ8 codes qs [t, k] and
    block scales sa [t, k/32]: every term f32(dot) * sw * sa is exact in f64 (a 15-bit integer
    dot, an 11-bit f16 scale and a 24-bit f32 scale), and so is their sum up to f64 rounding.
    Returns (y [t, n], R [t, n]) with R = sqrt(sum of squared terms), the scale of the partial
    sums an f32 accumulation walks through."""
    nb = k // 32
    w = blocks.reshape(n, nb)["qs"].astype(np.int64)                       # [n, nb, 32]
    sw = blocks.reshape(n, nb)["scale"].view(np.float16).astype(np.float64)  # [n, nb]
    q = np.asarray(qs, np.int64).reshape(-1, nb, 32)
    s = np.asarray(sa, np.float64).reshape(-1, nb)
    dots = np.einsum("nbj,tbj->tnb", w, q)
    terms = dots.astype(np.float64) * sw[None] * s[:, None, :]
    return terms.sum(axis=-1), np.sqrt((terms * terms).sum(axis=-1))


def q4_exact_terms(blocks, n, k, qs, sa):
    """As q8_exact_terms for BlockQ4 [n, k/32]: element 2j of a block is the low nibble of qs[j],
    element 2j+1 the high one, each a signed 4-bit code (crates/llm-quant/src/lib.rs:83-92)."""
    nb = k // 32
    raw = blocks.reshape(n, nb)["qs"].astype(np.int64)                        # [n, nb, 16]
    w = np.empty((n, nb, 32), np.int64)
    w[..., 0::2] = raw & 15
    w[..., 1::2] = raw >> 4
    w[w >= 8] -= 16
    sw = blocks.reshape(n, nb)["scale"].view(np.float16).astype(np.float64)
    q = np.asarray(qs, np.int64).reshape(-1, nb, 32)
    s = np.asarray(sa, np.float64).reshape(-1, nb)
    dots = np.einsum("nbj,tbj->tnb", w, q)
    terms = dots.astype(np.float64) * sw[None] * s[:, None, :]
    return terms.sum(axis=-1), np.sqrt((terms * terms).sum(axis=-1))


def summation_allowance(R, nterms):
    """What the order of an f32 summation of nterms terms can move the result by, at the scale R of
    its partial sums: 8 u sqrt(n) R with u = 2^-24 (the probabilistic rounding-error bound's form;
    8 standard deviations)."""
    return 8.0 * 2.0 ** -24 * np.sqrt(nterms) * np.asarray(R, np.float64)
