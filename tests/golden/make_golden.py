"""Write tests/golden/fixtures.npz: known-answer vectors for the Q4 / Q8_0 matmul path.

Run from the repository root:  python -m tests.golden.make_golden

The reference (Rust) cannot run here and holds no numeric golden vectors for
this path, so every expected value below is computed by an independent numpy
restatement of the reference's arithmetic -- not by the oracle -- and the
oracle is checked against it before anything is written:

  * BlockQ4::quantize / BlockQ8_0::quantize  crates/llm-quant/src/lib.rs:26-37, 63-79
  * ActQ8 (PerBlock / PerRow)                 crates/llm-cpu/src/gemv_q4.rs:33-95, 273-299
  * per-block integer dots                    crates/llm-cpu/src/gemv_q4.rs:959-966
  * gemv_tiles_scalar operation order         crates/llm-cpu/src/gemv_q4.rs:499-544
  * AddF64 epilogue                           crates/llm-cpu/src/gemv_q4.rs:486-497
  * q8_apply                                  crates/llm-engine/src/weights.rs:194-227

Inputs are the reference tests' formula-generated matrices (gemv_q4.rs:1080-1249,
amx.rs:526-557, llm-quant/src/lib.rs:149-222) plus hand-picked edge cases.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "fixtures.npz")

F32 = np.float32


# ---- numpy restatements ----------------------------------------------------------------
def round_half_away(v: np.ndarray) -> np.ndarray:
    """f32::round: exact, via trunc and the (exact) fractional part; inf and NaN pass through."""
    v = np.asarray(v, dtype=F32)
    with np.errstate(invalid="ignore"):
        t = np.trunc(v)
        frac = np.where(np.isfinite(v), v - t, F32(0))
        return (t + np.where(np.abs(frac) >= F32(0.5), np.sign(v), F32(0))).astype(F32)


def round_clamp_i8(v: np.ndarray, lo: float, hi: float) -> np.ndarray:
    """Rust `v.round().clamp(lo, hi) as i8`: clamp keeps NaN and `NaN as i8` is 0."""
    r = np.clip(round_half_away(v), lo, hi)
    return np.where(np.isnan(r), F32(0), r).astype(np.int8)


def act_quant_np(x: np.ndarray, per_row: bool):
    """ActQ8::quantize (gemv_q4.rs:62-95) / quantize_row (:37-60), row by row."""
    m, k = x.shape
    nb = k // 32
    qs = np.zeros((m, k), np.int8)
    sc = np.zeros((m, nb), F32)
    su = np.zeros((m, nb), np.int32)
    for r in range(m):
        row = x[r].astype(F32)
        if per_row:
            row_scale = F32(np.max(np.abs(row)) if k else 0) / F32(127)
        for b in range(nb):
            v = row[32 * b:32 * b + 32]
            scale = row_scale if per_row else F32(np.max(np.abs(v))) / F32(127)
            with np.errstate(over="ignore", invalid="ignore"):
                inv = F32(0) if scale == 0 else F32(1) / F32(scale)
                prod = v * inv
            q = round_clamp_i8(prod, -127, 127).astype(np.int32)
            qs[r, 32 * b:32 * b + 32] = q
            sc[r, b] = scale
            su[r, b] = q.sum()
    return qs, sc, su


def quantize_q4_np(x: np.ndarray):
    """BlockQ4::quantize: scale = f16(amax / 8), q = clamp(round(x / scale_f32), -8, 7)."""
    blocks = x.reshape(-1, 32).astype(F32)
    nib = np.zeros(blocks.shape, np.int8)
    bits = np.zeros(len(blocks), np.uint16)
    for i, v in enumerate(blocks):
        amax = F32(np.max(np.abs(v)))
        s16 = np.float16(amax / F32(8))
        s = F32(s16)
        inv = F32(0) if s == 0 else F32(1) / s
        nib[i] = round_clamp_i8(v * inv, -8, 7)
        bits[i] = s16.view(np.uint16)
    return nib, bits


def quantize_q8_np(x: np.ndarray):
    """BlockQ8_0::quantize: scale = f16(amax / 127), q = round(x / scale_f32) clamped to +-127."""
    blocks = x.reshape(-1, 32).astype(F32)
    q = np.zeros(blocks.shape, np.int8)
    bits = np.zeros(len(blocks), np.uint16)
    for i, v in enumerate(blocks):
        amax = F32(np.max(np.abs(v)))
        s16 = np.float16(amax / F32(127))
        s = F32(s16)
        inv = F32(0) if s == 0 else F32(1) / s
        q[i] = round_clamp_i8(v * inv, -127, 127)
        bits[i] = s16.view(np.uint16)
    return q, bits


def gemv_scalar_np(nib, wbits, n, k, qs, sa, add_to=None):
    """gemv_tiles_scalar: acc = acc + ((f32(idot) * sw) * sa) per block, ascending kb."""
    nb = k // 32
    w = nib.reshape(n, nb, 32).astype(np.int64)
    sw = wbits.view(np.float16).astype(F32).reshape(n, nb)
    idot = np.einsum("rbe,be->rb", w, qs.reshape(nb, 32).astype(np.int64))
    acc = np.zeros(n, F32)
    for b in range(nb):
        acc = (acc + (idot[:, b].astype(F32) * sw[:, b]) * F32(sa[b])).astype(F32)
    if add_to is not None:
        acc = (add_to.astype(np.float64) + acc.astype(np.float64)).astype(F32)
    return acc


def q8_apply_np(q, wbits, n, k, x):
    """q8_apply: ActQ8::quantize(x) per token, acc = acc + ((f32(dot) * f32(scale)) * sa)."""
    nb = k // 32
    qa, sa, _ = act_quant_np(x.reshape(1, k), False)
    w = q.reshape(n, nb, 32).astype(np.int64)
    sw = wbits.view(np.float16).astype(F32).reshape(n, nb)
    idot = np.einsum("rbe,be->rb", w, qa.reshape(nb, 32).astype(np.int64))
    acc = np.zeros(n, F32)
    for b in range(nb):
        acc = (acc + (idot[:, b].astype(F32) * sw[:, b]) * sa[0, b]).astype(F32)
    return acc


def pack_q4(nib, bits):
    from llmhost_amd.formats import q4_from_nibbles
    return q4_from_nibbles(nib, bits)


def formula(count, mul, mod, off, scale):
    return ((((np.arange(count) * mul) % mod) - off).astype(F32) * F32(scale)).astype(F32)


# ---- fixture content --------------------------------------------------------------------
def build() -> dict:
    fx = {}
    # ActQ8 edge rows: zero block, exact .5 ties, clamp, denormals, signed zeros, huge values.
    x = np.zeros((6, 128), F32)
    x[0, 32:40] = [127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -1.5, 3.5]
    x[1] = formula(128, 7, 15, 7, 0.2)
    x[2] = formula(128, 13, 19, 9, 0.15) * F32(1e-3)
    x[3, :32] = np.float32(1e-40) * np.arange(32, dtype=F32)      # denormal block
    x[3, 32:64] = -0.0
    x[3, 64:96] = F32(3.0e38) * np.sign(formula(32, 5, 11, 5, 1.0) + F32(0.5))
    x[4] = np.sin(np.arange(128, dtype=F32)).astype(F32) * F32(37.0)
    x[5] = formula(128, 3, 17, 8, 0.1) * F32(1e4)
    fx["act_x"] = x
    for tag, per_row in (("block", False), ("row", True)):
        qs, sc, su = act_quant_np(x, per_row)
        fx[f"act_qs_{tag}"], fx[f"act_sc_{tag}"], fx[f"act_sum_{tag}"] = qs, sc, su

    # Weight quantizers on the reference tests' formula weights (lib.rs:149-222).
    wf = np.concatenate([formula(32 * 9, 13, 19, 9, 0.15), formula(64, 3, 17, 8, 0.1),
                         np.zeros(32, F32), np.array([8.0, -8.0, 2.5, -2.5, 0.5, -0.5, 1.5, -7.5] * 4, F32)])
    fx["qw_x"] = wf
    fx["q4_nib"], fx["q4_bits"] = quantize_q4_np(wf)
    fx["q8_q"], fx["q8_bits"] = quantize_q8_np(wf)

    # Block dots: the reference's pattern_block seeds (gemv_q4.rs:1080-1102) + extremes.
    i = np.arange(32)
    dot_nib, dot_act = [], []
    for seed in range(16):
        w = (((i * 17 + seed) % 21) - 10).astype(F32) * F32(0.25)
        nib, _ = quantize_q4_np(w)
        dot_nib.append(nib[0])
        dot_act.append((((i * 9 + seed) % 25) - 12).astype(np.int8))
    dot_nib += [np.full(32, -8, np.int8), np.full(32, 7, np.int8), np.full(32, -8, np.int8)]
    dot_act += [np.full(32, -127, np.int8), np.full(32, 127, np.int8), np.full(32, 127, np.int8)]
    fx["dot_nib"] = np.stack(dot_nib)
    fx["dot_act"] = np.stack(dot_act)
    fx["dot_q4"] = np.einsum("be,be->b", fx["dot_nib"].astype(np.int64),
                             fx["dot_act"].astype(np.int64)).astype(np.int32)

    # GEMV / GEMM on the reference tests' formula inputs (gemv_q4.rs:1104-1249, amx.rs:526-557).
    for tag, n, k, wp, xp in (("a", 17, 64, (13, 19, 9, 0.15), (7, 15, 7, 0.2)),
                              ("b", 128, 64, (3, 17, 8, 0.1), (5, 11, 5, 0.2))):
        w = formula(n * k, *wp)
        xv = formula(k, *xp)
        nib, bits = quantize_q4_np(w)
        qs, sa, _ = act_quant_np(xv.reshape(1, k), False)
        fx[f"gemv_{tag}_w"], fx[f"gemv_{tag}_x"] = w, xv
        fx[f"gemv_{tag}_y"] = gemv_scalar_np(nib, bits, n, k, qs[0], sa[0])
        y0 = formula(n, 11, 23, 11, 3.0)
        fx[f"gemv_{tag}_y0"] = y0
        fx[f"gemv_{tag}_yadd"] = gemv_scalar_np(nib, bits, n, k, qs[0], sa[0], add_to=y0)
    n, k, m = 48, 64, 20
    w = ((((np.arange(n * k) * 3) % 17) - 8).astype(F32) * F32(0.1)).astype(F32)
    xm = ((((np.arange(m * k) * 5) % 11) - 5).astype(F32) * F32(0.2)).astype(F32).reshape(m, k)
    nib, bits = quantize_q4_np(w)
    qs, sa, _ = act_quant_np(xm, False)
    fx["gemm_w"], fx["gemm_x"] = w, xm
    fx["gemm_y"] = np.stack([gemv_scalar_np(nib, bits, n, k, qs[t], sa[t]) for t in range(m)])

    # Q8_0 head GEMV (q8_apply) on formula inputs.
    n, k = 33, 96
    w = formula(n * k, 13, 19, 9, 0.15)
    xv = formula(k, 7, 15, 7, 0.2)
    q, bits = quantize_q8_np(w)
    fx["q8_w"], fx["q8_x"] = w, xv
    fx["q8_y"] = q8_apply_np(q, bits, n, k, xv)
    return fx


def check_against_oracle(fx: dict) -> None:
    """The oracle must reproduce every vector (integers and the scalar-order floats exactly)."""
    import oracle

    for tag, per_row in (("block", False), ("row", True)):
        qs, sc, su = oracle.act_quantize(fx["act_x"], per_row)
        assert np.array_equal(qs, fx[f"act_qs_{tag}"]), tag
        assert np.array_equal(sc.view(np.uint32), fx[f"act_sc_{tag}"].view(np.uint32)), tag
        assert np.array_equal(su, fx[f"act_sum_{tag}"]), tag
    b4 = oracle.quantize_q4(fx["qw_x"])
    assert np.array_equal(b4.tobytes(), pack_q4(fx["q4_nib"], fx["q4_bits"]).tobytes())
    b8 = oracle.quantize_q8_0(fx["qw_x"])
    assert np.array_equal(b8["qs"], fx["q8_q"]) and np.array_equal(b8["scale"], fx["q8_bits"])
    blocks = pack_q4(fx["dot_nib"], np.full(len(fx["dot_nib"]), 0x3C00, np.uint16))
    got = [oracle.dot_q4_q8(blocks[j], fx["dot_act"][j]) for j in range(len(blocks))]
    assert np.array_equal(np.array(got, np.int32), fx["dot_q4"])
    for tag, n, k in (("a", 17, 64), ("b", 128, 64)):
        mat = oracle.Q4Matrix.from_f32(fx[f"gemv_{tag}_w"], n, k)
        y = oracle.gemv_q4(mat, fx[f"gemv_{tag}_x"], kernel=oracle.KERNEL_SCALAR)
        assert np.array_equal(y.view(np.uint32), fx[f"gemv_{tag}_y"].view(np.uint32)), tag
        ya = oracle.gemv_q4(mat, fx[f"gemv_{tag}_x"], out=fx[f"gemv_{tag}_y0"].copy(), add=True,
                            kernel=oracle.KERNEL_SCALAR)
        assert np.array_equal(ya.view(np.uint32), fx[f"gemv_{tag}_yadd"].view(np.uint32)), tag
    mat = oracle.Q4Matrix.from_f32(fx["gemm_w"], 48, 64)
    y = oracle.gemm_q4(mat, fx["gemm_x"], 20, kernel=oracle.KERNEL_SCALAR)
    assert np.array_equal(np.asarray(y).reshape(20, 48).view(np.uint32), fx["gemm_y"].view(np.uint32))
    b8 = oracle.quantize_q8_0(fx["q8_w"])
    y = oracle.q8_apply(b8, 33, 96, fx["q8_x"])
    assert np.array_equal(np.asarray(y).view(np.uint32), fx["q8_y"].view(np.uint32))


def main() -> None:
    sys.path.insert(0, ROOT)
    fx = build()
    check_against_oracle(fx)
    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(fx)} arrays)")


if __name__ == "__main__":
    main()
