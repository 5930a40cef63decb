"""Benchmark: Q4 GEMV HBM GB/s at M=1 (the headline) plus Q4 GEMM TOPS at M=512.

Headline workload (one "step"): the FFN-shaped Q4 decode GEMVs
  up   K=1536 -> N=8192   and   down K=8192 -> N=1536,
each launch reading a different copy of its weights from a rotating pool
larger than 2x the 256 MB Infinity Cache, so the bytes come from HBM.
x and y stay resident in HBM; fp32 x in, fp32 y out, activation
quantization fused into the GEMV.

value = algorithmic bytes / time, bytes = Q4 blocks as-is (18 B per 32
weights) + 4*K (x) + 4*N (y) per GEMV.

Also reported (one JSON line, under "extra"): the 16-layer decode sweep,
ragged Q4 GEMM M in {4,16,64}, prefill Q4 GEMM M=512 / 2048 TOPS (fraction of
int8 MFMA peak), Q8_0 GEMV K=N=1536, the tied heads, the decode FFN block
(fused vs per-op), the attention / conv block input side (norm + projections)
-- and, on rank 0, the CPU baseline: the
oracle's runtime-dispatched llm-cpu restatement (VNNI-512 > AVX2 > scalar)
timed on this host's cores over a bounded sample of the same GEMV workload.

Usage: python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu] [--quick]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
INT8_PEAK_TOPS = 5033.0        # MI355X dense int8 MFMA, TOPS (256 CU x 2.4 GHz x 8192)
MALL_BYTES = 256 << 20
METRIC = "Q4 GEMV HBM GB/s at M=1; Q4 GEMM TOPS at M=512 (frac. of roofline)"


def q4_bytes(n, k, m=1):
    return n * (k // 32) * 18 + 4 * k * m + 4 * n * m


def q8_bytes(n, k, m=1):
    return n * (k // 32) * 34 + 4 * k * m + 4 * n * m


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class GpuBench:
    def __init__(self):
        import torch

        from llmhost_amd import q4

        self.torch = torch
        self.q4 = q4
        self.ctx = q4.Context(0)
        self.stream = torch.cuda.Stream()  # default priority
        self.ctx.set_stream(self.stream.cuda_stream)

    def copies(self, n, k, seed, min_bytes):
        """Distinct device copies of one seeded Q4 matrix (uploaded once,
        re-packed on the device from a device-resident block buffer)."""
        from llmhost_amd import synth

        blocks = synth.q4_blocks(seed, n, k)
        raw = self.torch.from_numpy(blocks.view(np.uint8).copy()).cuda()
        per = n * (k // 32) * 18
        count = max(1, math.ceil(min_bytes / per))
        mats = [self.q4.Q4Matrix.from_blocks(n, k, raw, self.ctx) for _ in range(count)]
        del raw
        return blocks, mats

    def timed(self, fn, iters, warmup, reps=1):
        """ms per iteration of fn(i), i = 0..iters-1, replayed from a HIP graph (a list of `reps`
        such figures, one per replay, when reps > 1).

        The warm-up runs eagerly (it also sizes every workspace, so nothing is
        allocated under capture); the timed region is one replay of a graph
        holding all `iters` iterations, bracketed by device synchronisation
        and HIP events on the stream the library launches on.
        """
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for i in range(warmup):
                fn(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=self.stream):
            for i in range(iters):
                fn(i)
        # replay() launches on torch's current stream: make it the library's.
        samples = []
        with torch.cuda.stream(self.stream):
            graph.replay()  # first replay uploads the graph
            torch.cuda.synchronize()
            for _ in range(reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(self.stream)
                graph.replay()
                e1.record(self.stream)
                torch.cuda.synchronize()
                samples.append(e0.elapsed_time(e1) / iters)
        del graph
        return samples if reps > 1 else samples[0]  # ms per iteration


def gemv_workload(gb: GpuBench, steps: int, warmup: int):
    torch, q4 = gb.torch, gb.q4
    shapes = {"up": (8192, 1536), "down": (1536, 8192)}
    mats, xs, ys = {}, {}, {}
    for i, (name, (n, k)) in enumerate(shapes.items()):
        _, mats[name] = gb.copies(n, k, 101 + i, 2 * MALL_BYTES + (64 << 20))
        from llmhost_amd import synth

        xs[name] = torch.from_numpy(synth.normal_f32(201 + i, k)).cuda()
        ys[name] = torch.zeros(n, device="cuda")
    C = min(len(m) for m in mats.values())

    def step(i):
        q4.gemv_q4(mats["up"][i % C], xs["up"], ys["up"])
        q4.gemv_q4(mats["down"][i % C], xs["down"], ys["down"])

    ms = gb.timed(step, steps, warmup)
    step_bytes = sum(q4_bytes(n, k) for n, k in shapes.values())
    per_kernel = {}
    for name, (n, k) in shapes.items():
        def one(i, name=name):
            q4.gemv_q4(mats[name][i % C], xs[name], ys[name])
        kms = gb.timed(one, max(steps, 200), warmup)
        per_kernel[name] = {"n": n, "k": k, "us": kms * 1e3, "bytes": q4_bytes(n, k),
                            "gbs": q4_bytes(n, k) / (kms * 1e-3) / 1e9}
    return ms, step_bytes, C, per_kernel, mats


def launch_floor_and_read(gb: GpuBench, per_kernel, iters: int = 200):
    """What any launch of the headline GEMV's size can reach, timed in the same graph harness:
    the per-launch floor of dependent launches (the library's empty kernel at 1 and 256
    workgroups, and a one-element torch fill) and a plain streaming read of the GEMV's 7,116,800
    algorithmic bytes (the library's read probe at 1, 2, 4 and 8 loads per thread, and a torch
    row-sum reduction), each launch reading a different copy from a rotating pool > 2x MALL."""
    torch, q4 = gb.torch, gb.q4
    nbytes = q4_bytes(8192, 1536)
    assert nbytes == q4_bytes(1536, 8192) and nbytes % 1024 == 0
    count = math.ceil((2 * MALL_BYTES + (64 << 20)) / nbytes)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(17)
    bufs = [torch.randn(nbytes // 4, device="cuda", generator=gen) for _ in range(count)]
    out = torch.zeros(max(q4.probe_read_outputs(nbytes, u) for u in (1, 2, 4, 8)), device="cuda")
    rows = torch.zeros(nbytes // 4 // 256, device="cuda")
    tiny = torch.zeros(1, device="cuda")
    floor = {f"empty_{w}wg": gb.timed(lambda i, w=w: q4.probe_empty(w, gb.ctx), iters, 10) * 1e3
             for w in (1, 256)}
    floor["torch_fill_1"] = gb.timed(lambda i: tiny.fill_(1.0), iters, 10) * 1e3
    read = {f"probe_u{u}": gb.timed(lambda i, u=u: q4.probe_read(bufs[i % count], out, u, gb.ctx), iters, 10) * 1e3
            for u in (1, 2, 4, 8)}
    read["torch_row_sum"] = gb.timed(
        lambda i: torch.sum(bufs[i % count].view(-1, 256), dim=1, out=rows), iters, 10) * 1e3
    del bufs
    floor_us = min(floor["empty_1wg"], floor["empty_256wg"])
    read_us = min(v for k, v in read.items() if k.startswith("probe"))
    res = {"launch_floor_us": round(floor_us, 3), "stream_read_7MB_us": round(read_us, 3),
           "stream_read_7MB_gbs": round(nbytes / (read_us * 1e-6) / 1e9, 1), "bytes": nbytes,
           "copies": count, "floor_us": {k: round(v, 3) for k, v in floor.items()},
           "read_us": {k: round(v, 3) for k, v in read.items()}}
    for name, d in per_kernel.items():
        res[f"gemv_{name}_to_read"] = round(d["us"] / read_us, 3)
    return res


def decode_sweep(gb: GpuBench, iters: int):
    """16 layers: qkv 1536->2048, o 1536->1536, gate/up pair 1536->8192, down 8192->1536 (AddF64)."""
    torch, q4 = gb.torch, gb.q4
    from llmhost_amd import synth

    H, F, L = 1536, 8192, 16
    layers = []
    raw_cache = {}
    for layer in range(L):
        mats = {}
        for j, (name, n, k) in enumerate([("qkv", 2048, H), ("o", H, H), ("gate", F, H), ("up", F, H),
                                          ("down", H, F)]):
            key = (n, k, j)
            if key not in raw_cache:
                raw_cache[key] = torch.from_numpy(synth.q4_blocks(500 + j, n, k).view(np.uint8).copy()).cuda()
            mats[name] = q4.Q4Matrix.from_blocks(n, k, raw_cache[key], gb.ctx)
        layers.append(mats)
    raw_cache.clear()
    x = torch.from_numpy(synth.normal_f32(7, H)).cuda()
    qkv = torch.zeros(2048, device="cuda")
    h = torch.zeros(H, device="cuda")
    g = torch.zeros(F, device="cuda")
    u = torch.zeros(F, device="cuda")

    def step(_):
        for m in layers:
            q4.gemv_q4(m["qkv"], x, qkv)
            q4.gemv_q4(m["o"], x, h)
            q4.gemv_q4_pair(m["gate"], m["up"], x, g, u)
            q4.gemv_q4_add(m["down"], g, h)

    ms = gb.timed(step, iters, 2)
    total = L * (q4_bytes(2048, H) + q4_bytes(H, H) + 2 * q4_bytes(F, H) + q4_bytes(H, F))
    for m in layers:
        for w in m.values():
            w.free()
    return {"us": ms * 1e3, "bytes": total, "gbs": total / (ms * 1e-3) / 1e9,
            "frac_hbm": total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "launches": 4 * L}


def gemm_case(gb: GpuBench, m, n, k, iters, seed):
    torch, q4 = gb.torch, gb.q4
    from llmhost_amd import synth

    _, mats = gb.copies(n, k, seed, 2 * MALL_BYTES + (64 << 20))
    for w in mats:  # GEMM images up front: none may be built while the timed graph is captured
        w.prepare_gemm()
    x = torch.from_numpy(synth.activations(seed + 1, m, k)).cuda()
    y = torch.zeros(m, n, device="cuda")
    C = len(mats)
    samples = gb.timed(lambda i: q4.gemm_q4(mats[i % C], x, y, m), iters, 3, reps=5)
    ms = statistics.median(samples)
    ops = 2.0 * m * n * k
    byts = q4_bytes(n, k, m)
    for w in mats:
        w.free()
    return {"m": m, "n": n, "k": k, "us": ms * 1e3, "tops": ops / (ms * 1e-3) / 1e12,
            "frac_int8": ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, "gbs": byts / (ms * 1e-3) / 1e9,
            "samples_us": [round(t * 1e3, 3) for t in samples]}


def q8_case(gb: GpuBench, iters, n=1536, k=1536):
    """Q8_0 GEMV (q8_apply) over rotating copies (> 2x MALL)."""
    torch, q4 = gb.torch, gb.q4
    from llmhost_amd import synth

    b8 = synth.q8_blocks(71, n, k)
    count = math.ceil(2 * MALL_BYTES / (n * (k // 32) * 34))
    mats = [q4.Q8Matrix.from_blocks(n, k, b8, gb.ctx) for _ in range(count)]
    x = torch.from_numpy(synth.normal_f32(72, k)).cuda()
    y = torch.zeros(n, device="cuda")
    ms = gb.timed(lambda i: q4.q8_apply(mats[i % count], x, 1, y), iters, 10)
    for w in mats:
        w.free()
    return {"n": n, "k": k, "us": ms * 1e3, "gbs": q8_bytes(n, k) / (ms * 1e-3) / 1e9,
            "frac_hbm": q8_bytes(n, k) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}


def q8_head_norm_case(gb: GpuBench, iters, n=65536, k=1536):
    """The final rms_norm + Q8_0 head of a decode step (lfm2.rs:559-567): the norm fused into the
    head's GEMV against rms_norm then q8_apply.  Rotating copies > 2x MALL."""
    torch, q4 = gb.torch, gb.q4
    from llmhost_amd import synth

    b8 = synth.q8_blocks(71, n, k)
    count = math.ceil(2 * MALL_BYTES / (n * (k // 32) * 34))
    mats = [q4.Q8Matrix.from_blocks(n, k, b8, gb.ctx) for _ in range(count)]
    x = torch.from_numpy(synth.normal_f32(72, k)).cuda()
    nw = torch.from_numpy((1 + 0.1 * synth.normal_f32(73, k)).astype(np.float32)).cuda()
    normed = torch.zeros(k, device="cuda")
    y = torch.zeros(n, device="cuda")

    def sequence(i):
        q4.rms_norm(x, nw, 1e-5, normed, gb.ctx)
        q4.q8_apply(mats[i % count], normed, 1, y)

    ms_f = gb.timed(lambda i: q4.q8_norm_apply(mats[i % count], nw, 1e-5, x, 1, y), iters, 5)
    ms_s = gb.timed(sequence, iters, 5)
    for w in mats:
        w.free()
    byts = q8_bytes(n, k) + 4 * k
    return {"n": n, "k": k, "us": ms_f * 1e3, "gbs": byts / (ms_f * 1e-3) / 1e9,
            "frac_hbm": byts / (ms_f * 1e-3) / 1e9 / HBM_PEAK_GBS, "op_sequence_us": ms_s * 1e3}


def q4_head_case(gb: GpuBench, iters, n=65536, k=1536):
    """Q4 GEMV over rotating copies (> 2x MALL); default: the tied-head shape (the alternative to
    the Q8_0 head)."""
    torch, q4 = gb.torch, gb.q4
    from llmhost_amd import synth

    _, mats = gb.copies(n, k, 81, 2 * MALL_BYTES)
    x = torch.from_numpy(synth.normal_f32(82, k)).cuda()
    y = torch.zeros(n, device="cuda")
    C = len(mats)
    ms = gb.timed(lambda i: q4.gemv_q4(mats[i % C], x, y), iters, 5)
    for w in mats:
        w.free()
    return {"n": n, "k": k, "us": ms * 1e3, "gbs": q4_bytes(n, k) / (ms * 1e-3) / 1e9,
            "frac_hbm": q4_bytes(n, k) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}


def ffn_case(gb: GpuBench, iters, dim=1536, inter=8192):
    """Decode FFN residual block (lfm2.rs:883-911), one token: the fused two-launch entry point
    against the same math composed from the per-op entry points (torch for RMSNorm and
    silu * u).  Rotating weight sets > 2x MALL."""
    torch, q4 = gb.torch, gb.q4
    import torch.nn.functional as F
    from llmhost_amd import synth

    set_bytes = 2 * inter * (dim // 32) * 18 + dim * (inter // 32) * 18
    count = math.ceil(2 * MALL_BYTES / set_bytes)
    raws = [torch.from_numpy(synth.q4_blocks(600 + j, n, k).view(np.uint8).copy()).cuda()
            for j, (n, k) in enumerate([(inter, dim), (inter, dim), (dim, inter)])]
    sets = [[q4.Q4Matrix.from_blocks(n, k, raws[j], gb.ctx)
             for j, (n, k) in enumerate([(inter, dim), (inter, dim), (dim, inter)])] for _ in range(count)]
    del raws
    hidden = torch.from_numpy(synth.normal_f32(610, dim)).cuda()
    nw = torch.from_numpy((1 + 0.1 * synth.normal_f32(611, dim)).astype(np.float32)).cuda()
    g = torch.zeros(inter, device="cuda")
    u = torch.zeros(inter, device="cuda")

    def fused(i):
        w1, w3, w2 = sets[i % count]
        q4.ffn_residual(w1, w3, w2, nw, 1e-5, hidden)

    def unfused(i):
        w1, w3, w2 = sets[i % count]
        normed = nw * (hidden * torch.rsqrt((hidden.double() ** 2).mean() + 1e-5).float())
        q4.gemv_q4_pair(w1, w3, normed, g, u)
        h = F.silu(g) * u
        q4.gemv_q4_add(w2, h, hidden)

    def gemvs_only(i):  # the per-op path's two GEMV launches alone (no norm, no silu)
        w1, w3, w2 = sets[i % count]
        q4.gemv_q4_pair(w1, w3, hidden, g, u)
        q4.gemv_q4_add(w2, g, hidden)

    ms_f = gb.timed(fused, iters, 5)
    ms_u = gb.timed(unfused, iters, 5)
    ms_g = gb.timed(gemvs_only, iters, 5)
    for ws in sets:
        for w in ws:
            w.free()
    byts = set_bytes + 4 * dim * 3 + 4 * dim
    return {"dim": dim, "inter": inter, "us": ms_f * 1e3, "gbs": byts / (ms_f * 1e-3) / 1e9,
            "frac_hbm": byts / (ms_f * 1e-3) / 1e9 / HBM_PEAK_GBS, "unfused_us": ms_u * 1e3,
            "pair_and_down_gemvs_only_us": ms_g * 1e3,
            "bytes": byts, "launches": 2}


def ffn_prefill_case(gb: GpuBench, iters, dim=1536, inter=8192, tokens=512):
    """Prefill FFN residual block (lfm2.rs:861-881) over `tokens` rows: the entry point, whose
    gate/up activation image forms rms_norm(hidden) and whose down-projection image forms
    silu(g) * u, against the op sequence it replaces (rms_norm; the gate/up pair on one shared
    activation quantization; silu_mul; the down GEMM added in f64).  Rotating weight sets > 2x
    MALL, GEMM images built before capture; hidden accumulates the residual across calls (the
    norm keeps every call's input at unit RMS)."""
    torch, q4 = gb.torch, gb.q4
    from llmhost_amd import synth

    set_bytes = 2 * inter * (dim // 32) * 18 + dim * (inter // 32) * 18
    count = math.ceil((2 * MALL_BYTES + (64 << 20)) / set_bytes)
    shapes = [(inter, dim), (inter, dim), (dim, inter)]
    raws = [torch.from_numpy(synth.q4_blocks(620 + j, n, k).view(np.uint8).copy()).cuda()
            for j, (n, k) in enumerate(shapes)]
    sets = [[q4.Q4Matrix.from_blocks(n, k, raws[j], gb.ctx) for j, (n, k) in enumerate(shapes)]
            for _ in range(count)]
    del raws
    for ws in sets:
        for w in ws:
            w.prepare_gemm()
    hidden = torch.from_numpy(synth.activations(630, tokens, dim).ravel()).cuda()
    nw = torch.from_numpy((1 + 0.1 * synth.normal_f32(631, dim)).astype(np.float32)).cuda()
    normed = torch.zeros(tokens * dim, device="cuda")
    g = torch.zeros(tokens * inter, device="cuda")
    u = torch.zeros(tokens * inter, device="cuda")

    def fused(i):
        w1, w3, w2 = sets[i % count]
        q4.ffn_residual(w1, w3, w2, nw, 1e-5, hidden, tokens)

    def sequence(i):
        w1, w3, w2 = sets[i % count]
        q4.rms_norm(hidden, nw, 1e-5, normed, gb.ctx)
        q4.norm_gemv([w1, w3], None, 1e-5, normed, [g, u], tokens)
        q4.silu_mul(g, u, gb.ctx)
        q4.gemm_q4_add(w2, g, hidden, tokens)

    s_f = gb.timed(fused, iters, 3, reps=5)
    s_s = gb.timed(sequence, iters, 3, reps=5)
    for ws in sets:
        for w in ws:
            w.free()
    ms_f, ms_s = statistics.median(s_f), statistics.median(s_s)
    ops = 2.0 * tokens * dim * inter * 3
    return {"dim": dim, "inter": inter, "tokens": tokens, "us": ms_f * 1e3, "tops": ops / (ms_f * 1e-3) / 1e12,
            "frac_int8": ops / (ms_f * 1e-3) / 1e12 / INT8_PEAK_TOPS, "op_sequence_us": ms_s * 1e3,
            "samples_us": [round(t * 1e3, 3) for t in s_f], "op_sequence_samples_us": [round(t * 1e3, 3) for t in s_s]}


def block_input_case(gb: GpuBench, iters, rows, dim=1536, tokens=1):
    """Input side of an attention or conv block (lfm2.rs:784-794 / 651-659; prefill 698-711):
    rms_norm of `tokens` rows of hidden, then the block's projections (rows: the matrices' row
    counts, same K).  The entry point (one launch for a decode token; for several tokens one
    activation quantization shared by the matrices) against the op sequence (rms_norm, then one
    GEMV / GEMM per matrix).  Rotating weight sets > 2x MALL."""
    torch, q4 = gb.torch, gb.q4
    from llmhost_amd import synth

    set_bytes = sum(n * (dim // 32) * 18 for n in rows)
    count = math.ceil(2 * MALL_BYTES / set_bytes)
    raws = [torch.from_numpy(synth.q4_blocks(700 + j, n, dim).view(np.uint8).copy()).cuda()
            for j, n in enumerate(rows)]
    sets = [[q4.Q4Matrix.from_blocks(n, dim, raws[j], gb.ctx) for j, n in enumerate(rows)] for _ in range(count)]
    del raws
    if tokens > 64:  # the GEMM route: build every copy's GEMM image before the timed graph is captured
        for ws in sets:
            for w in ws:
                w.prepare_gemm()
    hidden = torch.from_numpy(synth.normal_f32(710, tokens * dim)).cuda()
    nw = torch.from_numpy((1 + 0.1 * synth.normal_f32(711, dim)).astype(np.float32)).cuda()
    normed = torch.zeros(tokens * dim, device="cuda")
    outs = [torch.zeros(tokens * n, device="cuda") for n in rows]

    def fused(i):
        q4.norm_gemv(sets[i % count], nw, 1e-5, hidden, outs, tokens)

    def sequence(i):
        q4.rms_norm(hidden, nw, 1e-5, normed, gb.ctx)
        for w, o in zip(sets[i % count], outs):
            q4.gemm_q4(w, normed, o, tokens)

    ms_f = gb.timed(fused, iters, 5)
    ms_s = gb.timed(sequence, iters, 5)
    for ws in sets:
        for w in ws:
            w.free()
    byts = set_bytes + 4 * dim * (tokens + 1) + 4 * tokens * sum(rows)
    ops = 2.0 * tokens * dim * sum(rows)
    return {"dim": dim, "rows": list(rows), "tokens": tokens, "us": ms_f * 1e3,
            "gbs": byts / (ms_f * 1e-3) / 1e9, "frac_hbm": byts / (ms_f * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "tops": ops / (ms_f * 1e-3) / 1e12, "op_sequence_us": ms_s * 1e3, "bytes": byts}


def decode_step_case(gb: GpuBench, iters, layers=16, dim=1536, inter=8192, vocab=65536):
    """The matmul side of a 16-layer decode step, chained as the engine runs it (lfm2.rs:559-567,
    784-911): per layer rms_norm + q / k / v (1536, 256, 256 rows: the sweep's qkv 1536x2048) in
    one launch, the output projection added onto hidden in f32 (its input stands in for the
    attention output: the layer's q), the fused FFN block; then the final rms_norm + Q8_0 head.
    Every call reads what the previous one wrote.  One weight set (391 MB of Q4 layers + 107 MB
    of head > 2x MALL, so each step streams from HBM)."""
    torch, q4 = gb.torch, gb.q4
    from llmhost_amd import synth

    raw = {}

    def mat(n, k, j):
        key = (n, k, j)
        if key not in raw:
            raw[key] = torch.from_numpy(synth.q4_blocks(800 + j, n, k).view(np.uint8).copy()).cuda()
        return q4.Q4Matrix.from_blocks(n, k, raw[key], gb.ctx)

    L = [{"q": mat(dim, dim, 0), "k": mat(256, dim, 1), "v": mat(256, dim, 2), "o": mat(dim, dim, 3),
          "w1": mat(inter, dim, 4), "w3": mat(inter, dim, 5), "w2": mat(dim, inter, 6)} for _ in range(layers)]
    raw.clear()
    head = q4.Q8Matrix.from_blocks(vocab, dim, synth.q8_blocks(810, vocab, dim), gb.ctx)
    nw = torch.from_numpy((1 + 0.1 * synth.normal_f32(811, dim)).astype(np.float32)).cuda()
    hidden0 = torch.from_numpy(synth.normal_f32(812, dim)).cuda()
    hidden = hidden0.clone()
    q, k, v = torch.zeros(dim, device="cuda"), torch.zeros(256, device="cuda"), torch.zeros(256, device="cuda")
    logits = torch.zeros(vocab, device="cuda")

    def step(_):
        hidden.copy_(hidden0)
        for m in L:
            q4.norm_gemv([m["q"], m["k"], m["v"]], nw, 1e-5, hidden, [q, k, v])
            q4.apply_add_inplace(m["o"], q, hidden)
            q4.ffn_residual(m["w1"], m["w3"], m["w2"], nw, 1e-5, hidden)
        q4.q8_norm_apply(head, nw, 1e-5, hidden, 1, logits)

    samples = gb.timed(step, iters, 2, reps=5)
    ms = float(np.median(samples))
    layer_bytes = sum(w.n * (w.k // 32) * 18 for w in L[0].values())
    total = layers * layer_bytes + vocab * (dim // 32) * 34
    for m in L:
        for w in m.values():
            w.free()
    head.free()
    return {"layers": layers, "us": ms * 1e3, "weight_bytes": total, "gbs": total / (ms * 1e-3) / 1e9,
            "frac_hbm": total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "launches": 4 * layers + 2,
            "tokens_per_s": 1e3 / ms, "samples_ms": [round(v, 5) for v in samples]}


def cpu_available() -> int:
    """CPUs this process may run on: its affinity mask, bounded by a cgroup CPU quota when one is
    set (a container's share of a larger host)."""
    n = len(os.sched_getaffinity(0))
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            n = min(n, max(1, int(quota) // int(period)))
    except (OSError, ValueError):
        pass
    return n


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _sys_jiffies():
    """(busy, total) jiffies of the whole machine from /proc/stat (bench/src/main.rs:103-117)."""
    with open("/proc/stat") as f:
        v = [int(t) for t in f.readline().split()[1:]]
    total = sum(v)
    return total - v[3] - (v[4] if len(v) > 4 else 0), total


def _own_jiffies():
    """utime + stime of this process (bench/src/main.rs:120-126)."""
    with open("/proc/self/stat") as f:
        rest = f.read().rsplit(")", 1)[1].split()
    return int(rest[11]) + int(rest[12])


def _loadavg():
    try:
        with open("/proc/loadavg") as f:
            return float(f.read().split()[0])
    except (OSError, ValueError):
        return float("nan")


def cpu_timed(fn, target_s: float):
    """Call fn() until target_s has passed; returns (calls, seconds, noise) with the reference's noise
    record (bench/src/main.rs:238-251): CPUs kept busy by other processes during the run."""
    load0, (b0, t0j), o0 = _loadavg(), _sys_jiffies(), _own_jiffies()
    t0 = time.perf_counter()
    calls = 0
    while True:
        fn(calls)
        calls += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    load1, (b1, t1j), o1 = _loadavg(), _sys_jiffies(), _own_jiffies()
    ncpu = len(os.sched_getaffinity(0))
    other = max(0.0, (b1 - b0) - (o1 - o0)) / max(1, t1j - t0j) * ncpu
    return calls, el, {"load_before": load0, "load_after": load1, "other_cpus": round(other, 3),
                       "noisy": other > 1.0}


def cpu_baseline(target_s: float = 10.0, row_s: float = 4.0):
    """The oracle's llm-cpu restatement (runtime-dispatched kernel: VNNI-512 > AVX2 > scalar, AMX
    tiles for the GEMM where the host has them; pinned pool of pool.rs) on this host, on 1 thread and on every available core (capped at
    pool.rs's 64), over rotating packed copies larger than the LLC: the headline GEMV step (the
    returned row), and rows for the M=512 prefill GEMM and the 16-layer decode sweep."""
    import oracle
    from llmhost_amd import synth

    cores = min(cpu_available(), oracle.lib().oq_max_threads())
    kern = oracle.detect_kernel()
    host = {"cpu_model": cpu_model(), "nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
            "available": cpu_available(), "kernel": oracle.kernel_name(kern)}
    rows = []

    # headline: up 1536 -> 8192 + down 8192 -> 1536 per step
    shapes = [(8192, 1536), (1536, 8192)]
    ncopies = 24  # 24 x 2 x 7.9 MB of packed CPU tiles, beyond a typical LLC
    mats, xs = [], []
    for i, (n, k) in enumerate(shapes):
        blocks = synth.q4_blocks(101 + i, n, k)
        mats.append([oracle.Q4Matrix(n, k, blocks) for _ in range(ncopies)])
        xs.append(synth.normal_f32(201 + i, k))
    outs = [np.zeros(n, dtype=np.float32) for n, _ in shapes]
    step_bytes = sum(q4_bytes(n, k) for n, k in shapes)
    headline = None
    for threads in (1, cores):
        def step(i, threads=threads):
            for s in range(2):
                oracle.gemv_q4(mats[s][i % ncopies], xs[s], outs[s], threads=threads)
        step(0)
        step(1)  # warm-up / page-in
        calls, el, noise = cpu_timed(step, target_s if threads == cores else row_s)
        gbs = calls * step_bytes / el / 1e9
        row = {"workload": "Q4 GEMV up K=1536,N=8192 + down K=8192,N=1536", "threads": threads,
               "value": round(gbs, 3), "unit": "GB/s", "frac_hbm_of_gpu": round(gbs / HBM_PEAK_GBS, 5),
               "ms_per_step": round(el / calls * 1e3, 4), "steps": calls, "seconds": round(el, 2), **noise}
        rows.append(row)
        if threads == cores:
            headline = (gbs, calls, el)
    del mats

    # prefill GEMM M=512, K=2048, N=10752 (4 rotating copies of 13.8 MB of tiles)
    m, n, k = 512, 10752, 2048
    blocks = synth.q4_blocks(912, n, k)
    gm = [oracle.Q4Matrix(n, k, blocks) for _ in range(4)]
    x = synth.activations(913, m, k)
    out = np.zeros((m, n), dtype=np.float32)
    # gemm_q4_mode (gemv_q4.rs:711) takes the AMX-INT8 tiles on a host that has them
    gemm_kern = oracle.kernel_name(oracle.KERNEL_AMX if oracle.amx_ready() else kern)
    for threads in (1, cores):
        oracle.gemm_q4(gm[0], x, m, out=out, threads=threads)
        calls, el, noise = cpu_timed(lambda i, t=threads: oracle.gemm_q4(gm[i % 4], x, m, out=out, threads=t), row_s)
        tops = calls * 2.0 * m * n * k / el / 1e12
        rows.append({"workload": f"Q4 GEMM M={m} K={k} N={n}", "threads": threads, "value": round(tops, 4),
                     "unit": "TOPS", "kernel": gemm_kern, "ms_per_call": round(el / calls * 1e3, 3), "calls": calls,
                     "seconds": round(el, 2), **noise})
    del gm

    # 16-layer decode sweep (qkv 1536->2048, o, gate/up pair 1536->8192, down 8192->1536 AddF64)
    H, F, L = 1536, 8192, 16
    layer_shapes = [("qkv", 2048, H), ("o", H, H), ("gate", F, H), ("up", F, H), ("down", H, F)]
    layers = [{name: oracle.Q4Matrix(n, kk, synth.q4_blocks(500 + j, n, kk))
               for j, (name, n, kk) in enumerate(layer_shapes)} for _ in range(L)]
    xh = synth.normal_f32(7, H)
    qkv, h = np.zeros(2048, np.float32), np.zeros(H, np.float32)

    def sweep(_i, threads):
        for lw in layers:
            oracle.gemv_q4(lw["qkv"], xh, qkv, threads=threads)
            oracle.gemv_q4(lw["o"], xh, h, threads=threads)
            g, u = oracle.gemv_q4_pair(lw["gate"], lw["up"], xh, threads=threads)
            oracle.gemv_q4(lw["down"], g, h, add=True, threads=threads)

    sweep_bytes = L * (q4_bytes(2048, H) + q4_bytes(H, H) + 2 * q4_bytes(F, H) + q4_bytes(H, F))
    for threads in (1, cores):
        sweep(0, threads)
        calls, el, noise = cpu_timed(lambda i, t=threads: sweep(i, t), row_s)
        rows.append({"workload": "Q4 decode sweep, 16 layers (391.6 MB)", "threads": threads,
                     "value": round(calls * sweep_bytes / el / 1e9, 3), "unit": "GB/s",
                     "tokens_per_s": round(calls / el, 3), "ms_per_step": round(el / calls * 1e3, 3),
                     "steps": calls, "seconds": round(el, 2), **noise})
    del layers

    gbs, calls, el = headline
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "kernel": oracle.kernel_name(kern),
            "sample": f"{calls} steps (up 1536->8192 + down 8192->1536 Q4 GEMV, fp32 x in, act-quant "
                      f"included) on {cores} pinned threads over {ncopies} rotating packed copies, {el:.1f} s",
            "ms_per_step": round(el / calls * 1e3, 4), "host": host, "rows": rows}


COUNTER_CASES = ("gemv", "gemm_m512_k2048", "gemm_m512_k10752", "ragged_m64", "copy")


def counters_mode(cases=COUNTER_CASES, iters: int = 50) -> None:
    """Eager launches for hardware-counter runs (rocprofv3 --pmc), one group per case:
    gemv: `iters` launches of each headline GEMV over rotating copies; gemm_m512_k2048 /
    gemm_m512_k10752: 5 prefill GEMM calls (M=512; K=2048, N=10752 / K=10752, N=2048);
    ragged_m64: 20 calls of the ragged M=64, K=2048, N=8192 GEMM; copy: a plain 64 MiB
    device-to-device copy (torch) of known size to calibrate FETCH_SIZE / WRITE_SIZE against.
    Prints the byte / op counts each kernel should move."""
    gb = GpuBench()
    torch, q4 = gb.torch, gb.q4
    from llmhost_amd import synth

    if "gemv" in cases:
        for i, (name, n, k) in enumerate([("up", 8192, 1536), ("down", 1536, 8192)]):
            _, mats = gb.copies(n, k, 101 + i, 2 * MALL_BYTES + (64 << 20))
            x = torch.from_numpy(synth.normal_f32(201 + i, k)).cuda()
            y = torch.zeros(n, device="cuda")
            with torch.cuda.stream(gb.stream):
                for it in range(iters):
                    q4.gemv_q4(mats[it % len(mats)], x, y)
            torch.cuda.synchronize()
            log(f"[counters] {name}: {iters} launches, algorithmic bytes/launch {q4_bytes(n, k)} "
                f"(weights {n * (k // 32) * 18})")
            for w in mats:
                w.free()
    for case, (m, n, k, calls) in (("gemm_m512_k2048", (512, 10752, 2048, 5)),
                                   ("gemm_m512_k10752", (512, 2048, 10752, 5)),
                                   ("ragged_m64", (64, 8192, 2048, 20))):
        if case not in cases:
            continue
        _, mats = gb.copies(n, k, 401 + k, 1)
        if m > 64:
            mats[0].prepare_gemm()
        x = torch.from_numpy(synth.activations(402, m, k)).cuda()
        y = torch.zeros(m, n, device="cuda")
        with torch.cuda.stream(gb.stream):
            for _ in range(calls):
                q4.gemm_q4(mats[0], x, y, m)
        torch.cuda.synchronize()
        log(f"[counters] {case} M={m} K={k} N={n}: {calls} calls, {2 * m * n * k} int8 ops and "
            f"{q4_bytes(n, k, m)} algorithmic bytes each")
        for w in mats:
            w.free()
    if "copy" in cases:
        src = torch.ones(16 << 20, device="cuda")
        dst = torch.empty_like(src)
        with torch.cuda.stream(gb.stream):
            for _ in range(iters):
                dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[counters] copy: {iters} launches of a 64 MiB read + 64 MiB write")


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4_gemv_hbm_traffic.txt")


def measured_traffic(name: str):
    """HBM bytes per launch of the headline GEMV `name` (up / down) from the
    committed PMC summary (FETCH_SIZE and WRITE_SIZE, copy-calibrated), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                parts = line.split()
                if len(parts) >= 3 and parts[0] == "traffic" and parts[1] == name:
                    return int(parts[2])
    except OSError:
        pass
    return None


KTRACE_FILE = os.path.join(ROOT, "profiles", "q4_gemv_up_down_k1536_n8192_kernel_trace.md")


def rocprof_avg_us(name: str):
    """Average kernel duration (us) of the headline GEMV `name` in the committed
    rocprofv3 kernel trace of `bench.py --quick`, or None."""
    try:
        with open(KTRACE_FILE) as f:
            for line in f:
                parts = line.split()
                if len(parts) >= 3 and parts[0] == "rocprof_avg_us" and parts[1] == name:
                    return float(parts[2])
    except (OSError, ValueError):
        pass
    return None


def roofline_entry(name: str, d: dict) -> dict:
    """The roofline object of the dominant GEMV `name`: `achieved` / `frac` from this run's HIP-event
    time of the kernel (graph-timed on the stream it is launched on); `frac_rocprof` from the average
    kernel duration of the committed rocprofv3 kernel trace; `traffic` (HBM bytes per launch) from the
    committed PMC summary -- the two file-sourced figures are named with their source, they are not
    measured in this run."""
    rp = rocprof_avg_us(name)
    return {"bound": "hbm", "kernel": f"q4_gemv ({name}: K={d['k']}, N={d['n']})",
            "achieved": round(d["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(d["gbs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(name),
            "bytes_per_launch": d["bytes"], "avg_launch_us": round(d["us"], 3),
            "rocprof_avg_us": rp,
            "frac_rocprof": round(d["bytes"] / (rp * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if rp else None,
            "sources": {"achieved": "this run, HIP events around a graph replay on the launch stream",
                        "traffic": os.path.relpath(TRAFFIC_FILE, ROOT) + " (rocprofv3 --pmc FETCH_SIZE + "
                                   "WRITE_SIZE per dispatch, copy-calibrated; not measured in this run)",
                        "rocprof_avg_us": os.path.relpath(KTRACE_FILE, ROOT) + " (rocprofv3 --kernel-trace "
                                          "--stats of bench.py --quick; not measured in this run)"}}


def _stats(xs):
    xs = sorted(xs)
    mean = sum(xs) / len(xs)
    sd = math.sqrt(sum((v - mean) ** 2 for v in xs) / max(1, len(xs) - 1)) if len(xs) > 1 else 0.0
    return {"tok_s_mean": mean, "tok_s_stdev": sd, "tok_s_p50": xs[len(xs) // 2], "tok_s_min": xs[0],
            "tok_s_max": xs[-1]}


def _git(*args):
    import subprocess

    try:
        return subprocess.run(["git", *args], cwd=ROOT, capture_output=True, text=True, timeout=10).stdout.strip()
    except (OSError, subprocess.SubprocessError):
        return ""


def jsonl_rows(extra, cpu):
    """Decode rows in the reference benchmark's JSONL schema (bench/src/main.rs:255-266): test "tg1"
    is one decode token through the 16-layer matmul stack (the engine's mixing steps are not on
    this path), tokens/s per sample."""
    common = {"commit": _git("rev-parse", "--short", "HEAD"), "dirty": bool(_git("status", "--porcelain")),
              "cpu": cpu_model(), "unix_time": int(time.time())}
    rows = []
    step = extra.get("decode_step_16L_chained")
    if step:
        xs = [1e3 / v for v in step["samples_ms"]]
        rows.append({"engine": "llm-gpu-hip", "model": "LFM2-700M-shaped 16-layer matmul stack (synthetic)",
                     "weights": "Q4_32 + Q8_0 head", "test": "tg1", "threads": None, "device": "MI355X",
                     "runs": len(xs), **_stats(xs), "samples": xs, "load_before": None, "load_after": None,
                     "other_cpus": None, "noisy": False, **common})
    for r in (cpu or {}).get("rows", []):
        if "tokens_per_s" not in r:
            continue
        xs = [r["tokens_per_s"]]
        rows.append({"engine": "llm-cpu (oracle restatement)", "model": "16-layer Q4 decode sweep (synthetic)",
                     "weights": "Q4_32", "test": "tg1", "threads": r["threads"], "runs": 1, **_stats(xs),
                     "samples": xs, "load_before": r["load_before"], "load_after": r["load_after"],
                     "other_cpus": r["other_cpus"], "noisy": r["noisy"], **common})
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--quick", action="store_true", help="headline GEMV only")
    ap.add_argument("--counters", nargs="?", const=",".join(COUNTER_CASES), default=None,
                    help="eager launches for rocprofv3 --pmc runs (no JSON line); optionally a comma-separated "
                         f"subset of {','.join(COUNTER_CASES)}")
    ap.add_argument("--only", default=None,
                    help="comma-separated extra rows to run alone (no headline, no CPU baseline), e.g. for "
                         "a per-shape kernel trace")
    ap.add_argument("--jsonl", default=None,
                    help="also append decode rows in the reference benchmark's JSONL schema to this file")
    args = ap.parse_args()
    if args.counters:
        cases = args.counters.split(",")
        unknown = set(cases) - set(COUNTER_CASES)
        if unknown:
            print(f"bench.py --counters: unknown cases {sorted(unknown)}", file=sys.stderr)
            sys.exit(2)
        counters_mode(cases)
        return
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported (the hot path is a "
              "single-GPU kernel; a multi-GPU split would shard weight rows by N and is not "
              "built)", file=sys.stderr)
        sys.exit(2)

    # Every `extra` row: (key, progress label, function; `gb` is bound below).  --only runs the
    # named rows alone (for per-shape kernel traces and counters) and skips the headline.
    sections = [("decode_sweep_16L", "decode sweep", lambda: decode_sweep(gb, 10))]
    for m in (4, 16, 64):
        sections.append((f"ragged_gemm_m{m}", f"ragged gemm M={m}", lambda m=m: gemm_case(gb, m, 8192, 2048, 50, 300 + m)))
    for (m, n, k) in [(512, 10752, 2048), (512, 2048, 10752), (2048, 10752, 2048), (2048, 2048, 10752)]:
        sections.append((f"prefill_gemm_m{m}_k{k}_n{n}", f"prefill gemm M={m} K={k} N={n}",
                         lambda m=m, n=n, k=k: gemm_case(gb, m, n, k, 10, 400 + m + k)))
    sections.append(("gemm_m_sweep_k2048_n8192", "Q4 GEMM M sweep across the route boundaries (K=2048, N=8192)",
                     lambda: [{k2: round(v, 3) if isinstance(v, float) else v
                               for k2, v in gemm_case(gb, m, 8192, 2048, 20, 900 + m).items() if k2 != "samples_us"}
                              for m in (32, 48, 49, 56, 64, 65, 72, 80, 96, 97, 112, 128)]))
    sections += [
        ("q8_gemv_k1536_n1536", "q8 gemv", lambda: q8_case(gb, 200)),
        ("q4_gemv_k1536_n1536", "Q4 GEMV K=N=1536 (the target's smallest shape)",
         lambda: q4_head_case(gb, 200, 1536, 1536)),
        ("q8_head_k1536_n65536", "tied head (N=65536, K=1536): Q8_0", lambda: q8_case(gb, 20, 65536, 1536)),
        ("final_norm_q8_head_k1536_n65536", "final norm + Q8_0 head", lambda: q8_head_norm_case(gb, 20)),
        ("decode_step_16L_chained", "chained 16-layer decode step (fused entry points)",
         lambda: decode_step_case(gb, 10)),
        ("q4_head_k1536_n65536", "tied head (N=65536, K=1536): Q4", lambda: q4_head_case(gb, 20)),
        ("q4_gemv_size_sweep", "Q4 GEMV size sweep (launch floor -> HBM bound)", lambda: [
            {k: round(v, 3) if isinstance(v, float) else v for k, v in q4_head_case(gb, 40, n, k).items()}
            for (n, k) in ((8192, 1536), (16384, 1536), (32768, 1536), (65536, 1536), (131072, 1536),
                           (1536, 8192), (4096, 8192), (16384, 8192))]),
        ("ffn_block_dim1536_inter8192", "decode FFN block (fused vs per-op)", lambda: ffn_case(gb, 100)),
        ("attn_qkv_dim1536", "attention block input side (norm + q/k/v, fused vs op sequence)",
         lambda: block_input_case(gb, 100, (1536, 512, 512))),
        ("conv_in_proj_dim1536", "conv block input side (norm + in_proj)", lambda: block_input_case(gb, 100, (4608,))),
        ("attn_qkv_dim1536_prefill_m512", "attention block input side, 512 tokens",
         lambda: block_input_case(gb, 10, (1536, 512, 512), tokens=512)),
        ("ffn_block_dim1536_inter8192_prefill_m512",
         "prefill FFN block (norm and silu * u fused into the activation images vs op sequence)",
         lambda: ffn_prefill_case(gb, 10)),
    ]
    only = set(args.only.split(",")) if args.only else None
    if only:
        unknown = only - {key for key, _, _ in sections}
        if unknown:
            print(f"bench.py --only: unknown rows {sorted(unknown)}", file=sys.stderr)
            sys.exit(2)
    gb = GpuBench()
    if only:
        extra = {}
        for key, label, fn in sections:
            if key in only:
                log(f"[bench] {label}")
                extra[key] = fn()
        print(json.dumps({"metric": METRIC, "only": sorted(only), "extra": extra}), flush=True)
        return
    log("[bench] headline GEMV workload")
    ms, step_bytes, copies, per_kernel, _ = gemv_workload(gb, args.steps, args.warmup)
    value = step_bytes / (ms * 1e-3) / 1e9
    dom = min(per_kernel.values(), key=lambda d: d["gbs"])
    dom_name = [k for k, v in per_kernel.items() if v is dom][0]
    extra = {"gemv_per_kernel": per_kernel, "weight_copies_per_shape": copies}
    log("[bench] launch floor and plain 7.1 MB read (same harness)")
    extra["launch_floor_and_read"] = launch_floor_and_read(gb, per_kernel)
    if not args.quick:
        for key, label, fn in sections:
            log(f"[bench] {label}")
            extra[key] = fn()
    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline")
        cpu = cpu_baseline()
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded SplitMix64: uniform Q4 nibbles, f16 scales U[1e-3,2e-2], x ~ N(0,1))",
        "config": {"workload": "Q4 GEMV M=1: up K=1536,N=8192 + down K=8192,N=1536 per step, "
                               f"{copies} rotating weight copies per shape (> 2x MALL)",
                   "global_batch": 1, "seq_len": 1, "parallelism": "single GPU"},
        "roofline": roofline_entry(dom_name, dom),
        "cpu_baseline": cpu,
        "extra": extra,
    }
    if "prefill_gemm_m512_k2048_n10752" in extra:
        g = extra["prefill_gemm_m512_k2048_n10752"]
        out["gemm_m512"] = {"tops": round(g["tops"], 2), "frac_int8_peak": round(g["frac_int8"], 4),
                            "us": round(g["us"], 2),
                            "roofline": {"bound": "mfma", "achieved": round(g["tops"], 2),
                                         "peak": INT8_PEAK_TOPS, "unit": "TOPS (int8 dense)",
                                         "frac": round(g["frac_int8"], 4)}}
    if args.jsonl:
        with open(args.jsonl, "a") as f:
            for row in jsonl_rows(extra, cpu):
                f.write(json.dumps(row) + "\n")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
