"""A chained decode step through the engine-level entry points against the oracle composing the
same reference ops (crates/llm-engine/src/lfm2.rs:519-573, 784-911).

Per layer: rms_norm + q / k / v (lgh_q4_norm_gemv, one launch), the output projection added onto
hidden in f32 (LGH_ADD_F32; its input stands in for the attention output: the layer's q), the
fused FFN block (lgh_q4_ffn_residual); then the final rms_norm + Q8_0 head (lgh_q8_norm_gemv).
Every call reads, on the device, what the previous call wrote.  Two layers, and the 16 of the
benchmark's chained step (hidden 1536, ffn 8192, q/k/v 1536/256/256 rows, vocab 65536), with
distinct weights per layer.

Gate: each call, re-anchored on the device's own input to it, matches the oracle's op within the
output tolerance (the FFN block with the allowance for the h codes an ulp of exp can flip, and the
f32 residual add with two ulps of its sum).  The oracle's un-anchored composition of the whole
step is compared as a sanity check: a flipped code moves one term of one block by at most
|nibble| * sw * sa, so the step's logits stay within 1e-3 of their scale.
"""

import numpy as np
import pytest

from llmhost_amd import q4, synth

from .conftest import ATOL, RTOL, assert_close, assert_close_with_flips, code_flip_bound

pytestmark = pytest.mark.gpu

DIM, INTER, KV, VOCAB = 1536, 8192, 256, 65536


def _ulp(a):
    return np.spacing(np.abs(np.asarray(a, np.float32))).astype(np.float64)


@pytest.mark.parametrize("n_layers", [2, 16])
def test_chained_decode_step(gpu_ctx, oracle, n_layers):
    import torch

    rng_seed = 900
    shapes = {"q": (DIM, DIM), "k": (KV, DIM), "v": (KV, DIM), "o": (DIM, DIM), "w1": (INTER, DIM),
              "w3": (INTER, DIM), "w2": (DIM, INTER)}
    layers = []
    for li in range(n_layers):
        L = {}
        for j, (name, (n, k)) in enumerate(shapes.items()):
            b = synth.q4_blocks(rng_seed + 10 * li + j, n, k)
            L[name] = (b, q4.Q4Matrix.from_blocks(n, k, b, gpu_ctx), oracle.Q4Matrix(n, k, b))
        L["nw_attn"] = (1 + 0.1 * synth.normal_f32(rng_seed + 10 * li + 8, DIM)).astype(np.float32)
        L["nw_ffn"] = (1 + 0.1 * synth.normal_f32(rng_seed + 10 * li + 9, DIM)).astype(np.float32)
        layers.append(L)
    hb = synth.q8_blocks(rng_seed + 99, VOCAB, DIM)
    head = q4.Q8Matrix.from_blocks(VOCAB, DIM, hb, gpu_ctx)
    nw_final = (1 + 0.1 * synth.normal_f32(rng_seed + 98, DIM)).astype(np.float32)
    hidden0 = (synth.normal_f32(rng_seed + 97, DIM) * np.float32(2.0)).astype(np.float32)

    # ---- the step on the device, every intermediate kept (copied to the host after the step)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    hidden = dev(hidden0)
    trace = []
    for L in layers:
        h_in = hidden.clone()
        q, k, v = (torch.zeros(n, device="cuda") for n in (DIM, KV, KV))
        q4.norm_gemv([L["q"][1], L["k"][1], L["v"][1]], dev(L["nw_attn"]), 1e-5, hidden, [q, k, v])
        q4.apply_add_inplace(L["o"][1], q, hidden)
        h_mid = hidden.clone()
        q4.ffn_residual(L["w1"][1], L["w3"][1], L["w2"][1], dev(L["nw_ffn"]), 1e-5, hidden)
        trace.append({"in": h_in, "q": q, "k": k, "v": v, "mid": h_mid, "out": hidden.clone()})
    logits = torch.zeros(VOCAB, device="cuda")
    q4.q8_norm_apply(head, dev(nw_final), 1e-5, hidden, 1, logits)
    torch.cuda.synchronize()
    trace = [{key: t.cpu().numpy() for key, t in st.items()} for st in trace]
    logits = logits.cpu().numpy()
    assert np.array_equal(trace[0]["in"], hidden0)

    # ---- gate: every call, re-anchored on the device's input to it
    for li, (L, st) in enumerate(zip(layers, trace)):
        normed = oracle.rms_norm(st["in"], L["nw_attn"], 1e-5)
        for name in ("q", "k", "v"):
            assert_close(st[name], oracle.gemv_q4(L[name][2], normed, threads=8), what=f"layer {li} {name}")
        y = oracle.gemv_q4(L["o"][2], st["q"], threads=8)
        ref_mid = (st["in"] + y).astype(np.float32)  # apply, then add_inplace in f32 (ops.rs:48-53)
        assert_close_with_flips(st["mid"], ref_mid, 2 * _ulp(ref_mid) + RTOL * np.abs(y),
                                what=f"layer {li} out-proj + residual")
        # FFN: the codes of the device's own h against the oracle's, as in the block test
        _, _, _, hq, hs = q4.ffn_gate_up(L["w1"][1], L["w3"][1], L["nw_ffn"], 1e-5, st["mid"])
        n2 = oracle.rms_norm(st["mid"], L["nw_ffn"], 1e-5)
        rg, ru = oracle.gemv_q4_pair(L["w1"][2], L["w3"][2], n2, threads=8)
        q_ref, s_ref, _ = oracle.act_quantize(oracle.silu_mul(rg, ru).reshape(1, -1), False)
        ref_out = oracle.ffn_residual(L["w1"][2], L["w3"][2], L["w2"][2], L["nw_ffn"], 1e-5, st["mid"], threads=8)
        bound, flips, _ = code_flip_bound(L["w2"][0], DIM, INTER, q_ref.ravel(), s_ref.ravel(), hq, hs)
        assert flips <= INTER // 500, f"layer {li}: {flips} h codes differ"
        assert_close_with_flips(st["out"], ref_out, bound, what=f"layer {li} ffn ({flips} flips)")
        if li + 1 < n_layers:
            assert np.array_equal(trace[li + 1]["in"], st["out"])
    ref_logits = oracle.q8_apply(hb, VOCAB, DIM, oracle.rms_norm(trace[-1]["out"], nw_final, 1e-5), 1, threads=8)
    assert_close(logits, ref_logits, what="final norm + q8 head")

    # ---- the oracle's own composition of the whole step, not re-anchored
    h = hidden0.copy()
    for L in layers:
        normed = oracle.rms_norm(h, L["nw_attn"], 1e-5)
        qq = oracle.gemv_q4(L["q"][2], normed, threads=8)
        h = (h + oracle.gemv_q4(L["o"][2], qq, threads=8)).astype(np.float32)
        h = oracle.ffn_residual(L["w1"][2], L["w3"][2], L["w2"][2], L["nw_ffn"], 1e-5, h, threads=8)
    full = oracle.q8_apply(hb, VOCAB, DIM, oracle.rms_norm(h, nw_final, 1e-5), 1, threads=8)
    scale = np.abs(full).max()
    err = np.abs(logits.astype(np.float64) - full)
    assert err.max() <= ATOL + 1e-3 * scale, (err.max(), scale)
    for w in [L[n][1] for L in layers for n in shapes] + [head]:
        w.free()
