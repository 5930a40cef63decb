"""Seeded random shapes through every device route, against the exact sum of the same ActQ8 codes.

Each case draws N, K, M and the mode from a fixed seed (so a failure names a reproducible case),
runs one entry point -- gemm_q4 / gemm_q4_add / the f32 residual add (the GEMV, batch,
matrix-core and GEMM routes by M), the norm GEMV over 1-3 matrices, the gate/up pair, the
prepared-activation GEMV or the Q8_0 GEMV -- and checks every output against the exact value of
the same block terms (each term f32(dot) * sw * sa is exact in f64, gemv_q4.rs:659-661,
weights.rs:206-212) within the output gate plus the f32 summation allowance of the block count.
"""

import numpy as np
import pytest

from llmhost_amd import _ffi, q4, synth

from .conftest import q4_exact_terms, q8_exact_terms, summation_allowance

pytestmark = pytest.mark.gpu

CASES = 160


def _within(dev, exact, R, nb, extra=0.0):
    allow = summation_allowance(R, nb) + 1e-4 + 1e-5 * np.abs(exact) + extra
    err = np.abs(np.asarray(dev, np.float64) - exact)
    bad = err > allow
    assert np.isfinite(dev).all()
    assert not bad.any(), f"{int(bad.sum())} of {bad.size} out of bound, max err {err.max():.3e}"


def _case(rng):
    r = rng.random()
    m = int(rng.integers(1, 5)) if r < 0.3 else int(rng.integers(5, 65)) if r < 0.6 else \
        int(rng.integers(65, 300)) if r < 0.9 else int(rng.integers(300, 700))
    r = rng.random()
    k = 32 * (int(rng.integers(1, 130)) if r < 0.6 else int(rng.integers(130, 400)) if r < 0.9 else
              int(rng.integers(1000, 1100)))
    n = int(rng.integers(1, 2500))
    while n > 1 and m * n * (k // 32) > 6_000_000:  # exact sums stay small on the host
        n //= 2
    kind = str(rng.choice(["gemm", "gemm", "gemm", "norm", "q8", "pair", "prep"]))
    mode = int(rng.choice([_ffi.LGH_ASSIGN, _ffi.LGH_ADD_F64, _ffi.LGH_ADD_F32]))
    return kind, n, k, m, bool(rng.random() < 0.25), mode, int(rng.integers(1 << 30))


def test_random_shapes_every_route(gpu_ctx, oracle):
    rng = np.random.default_rng(20251202)
    for i in range(CASES):
        kind, n, k, m, per_row, mode, seed = _case(rng)
        print(f"[fuzz {i}] {kind} n={n} k={k} m={m} per_row={per_row} mode={mode} seed={seed}", flush=True)
        if kind == "q8":
            t = 1 + m % 5
            b8 = synth.q8_blocks(seed, n, k)
            w8 = q4.Q8Matrix.from_blocks(n, k, b8, gpu_ctx)
            x = synth.activations(seed + 1, t, k)
            got = np.zeros(t * n, np.float32)
            q4.q8_apply(w8, x, t, got)
            qs, sa, _ = oracle.act_quantize(x, False)
            exact, R = q8_exact_terms(b8, n, k, qs, sa)
            _within(got.reshape(t, n), exact, R, k // 32)
            w8.free()
            continue
        blocks = synth.q4_blocks(seed, n, k)
        w = q4.Q4Matrix.from_blocks(n, k, blocks, gpu_ctx)
        x = synth.activations(seed + 1, m, k)
        gpu_ctx.set_act_quant(q4.ActQuant.PerRow if per_row else q4.ActQuant.PerBlock)
        try:
            if kind == "gemm":
                y0 = synth.activations(seed + 2, m, n)
                got = np.zeros((m, n), np.float32) if mode == _ffi.LGH_ASSIGN else y0.copy()
                if mode == _ffi.LGH_ASSIGN:
                    q4.gemm_q4(w, x, got, m) if m > 1 else q4.gemv_q4(w, x[0], got[0])
                elif mode == _ffi.LGH_ADD_F64:
                    q4.gemm_q4_add(w, x, got, m) if m > 1 else q4.gemv_q4_add(w, x[0], got[0])
                else:
                    q4.apply_add_inplace(w, x, got, m)
                qs, sa, _ = oracle.act_quantize(x, per_row)
                exact, R = q4_exact_terms(blocks, n, k, qs, sa)
                extra = 0.0
                if mode != _ffi.LGH_ASSIGN:  # the add rounds the sum once more, to f32
                    exact = exact + y0.astype(np.float64)
                    extra = np.abs(exact) * 2.0 ** -23
                _within(got, exact, R, k // 32, extra)
            elif kind == "norm":
                nm = 1 + seed % 3
                mats, outs, bl = [w], [np.zeros((m, n), np.float32)], [blocks]
                for j in range(1, nm):
                    nj = 1 + (seed >> (4 * j)) % 1500
                    bj = synth.q4_blocks(seed + 10 + j, nj, k)
                    mats.append(q4.Q4Matrix.from_blocks(nj, k, bj, gpu_ctx))
                    bl.append(bj)
                    outs.append(np.zeros((m, nj), np.float32))
                nw = (1 + 0.1 * synth.normal_f32(seed + 3, k)).astype(np.float32)
                q4.norm_gemv(mats, nw, 1e-5, x, outs, tokens=m)
                xn = oracle.rms_norm(x, nw, 1e-5).reshape(m, k)
                qs, sa, _ = oracle.act_quantize(xn, per_row)
                for j in range(nm):
                    exact, R = q4_exact_terms(bl[j], mats[j].n, k, qs, sa)
                    _within(outs[j], exact, R, k // 32)
                for mm in mats[1:]:
                    mm.free()
            elif kind == "pair":
                b2 = synth.q4_blocks(seed + 5, n, k)
                w2 = q4.Q4Matrix.from_blocks(n, k, b2, gpu_ctx)
                g, u = np.zeros(n, np.float32), np.zeros(n, np.float32)
                q4.gemv_q4_pair(w, w2, x[0], g, u)
                qs, sa, _ = oracle.act_quantize(x[:1], per_row)
                for dev, bb in ((g, blocks), (u, b2)):
                    exact, R = q4_exact_terms(bb, n, k, qs, sa)
                    _within(dev[None], exact, R, k // 32)
                w2.free()
            else:  # prep: codes and scales handed in, any act-quant mode's
                qs, sa, _ = oracle.act_quantize(x[:1], per_row)
                acts = q4.ActQ8(qs[0].copy(), sa[0].copy(), np.zeros(k // 32, np.int32))
                got = np.zeros(n, np.float32)
                q4.gemv_q4_prep(w, acts, got)
                exact, R = q4_exact_terms(blocks, n, k, qs, sa)
                _within(got[None], exact, R, k // 32)
        finally:
            gpu_ctx.set_act_quant(q4.ActQuant.PerBlock)
            w.free()
    gpu_ctx.trim()
