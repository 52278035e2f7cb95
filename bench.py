#!/usr/bin/env python3
"""Benchmark of the quantized matmul path on one MI355X.

Headline (the `value`): greedy decode tokens/s of a random-init 1.8B 2Bit
model (32 layers, hidden 2048, 16/4 heads of 128, SwiGLU 6144, Q2_0C
linears, tied Q6_K embedding/lm_head of 120818 rows, RMSNorm eps 1e-5, RoPE
base 11158840) with an f32 KV cache pre-filled to 1024 positions of N(0,1).
A step is one decode token (one replay of the captured HIP graph of the
whole forward pass plus argmax); warmup W and timed K steps run at positions
1024 .. 1024+W+K-1 (128 positions at the defaults).

Also reported, from live HIP-event timings on the context stream:
  roofline        the kernel with the largest time share of a decode step among
                  those decode_kernels times as the very instantiation the step
                  launches (the step's attention launch: RoPE, q/k norms, KV
                  append and split softmax partials over the 1032 cached
                  positions, K/V rotated over 64 layer caches so that they come
                  from HBM), launched alone through the C ABI: algorithmic bytes
                  per launch / average launch time (HIP events on the context
                  stream); `traffic` and `fetch_bytes` are the counter-measured
                  HBM bytes per launch of the same kernel
                  (profiles/*_traffic.json);
  step_hbm        the bytes a token streams (weights + KV cache) / time per token;
  device_copy_GBs (in roofline) a 1 GiB device-to-device copy's read + write
                  bytes / time;
  read_ceiling_GBs (in roofline) a read-only stream of a 2 GiB buffer: the
                  practical ceiling of the HBM-bound (read-dominated) kernels;
  decode_kernels  the step's other kernels timed the same way;
  gemv            GB/s of every matrix of the GEMV workloads (Q4_K [6144x2048];
                  the 1.8B Q2_0C/STQ1_0 set; Q6_K lm_head; the 7B shapes, and
                  the 7B gate/up pair as the step launches it: one fused
                  SiLU launch of both [14336 x 4096] matrices), Q8 input,
                  weights rotated over >= 1 GiB of distinct copies:
                  back-to-back launches, and (graph_GBs) one HIP graph that
                  launches every copy once, each beside a read-only launch of
                  the same bytes; for STQ1_0 the synthetic codes' measured zero
                  fraction;
  decode_models   the same decode measurement for the 1.8B 1.25Bit (STQ1_0)
                  model and a 7B Q4_K_M model (hidden 4096, 32/8 heads, FFN
                  14336, Q4_K linears, Q6_K down and tied embedding/lm_head of
                  128167 rows): tok/s and step_hbm;
  prefill, moe    the batched f16-MFMA GEMM (TFLOP/s) and the MoE expert layer;
                  mfma_ceiling (in prefill) the sustained rate of back-to-back
                  independent f16 MFMAs on every CU: the practical ceiling of
                  the GEMMs (of_mfma_ceiling);
  prefill_1p8b    the same model's chunked prefill of a 1024-token prompt
                  (hyq_dense_prefill), wall-clock tok/s;
  cpu_baseline    the reference's x86 decode step (f32 activations, scalar
                  Q2_0C row dot, AVX2 dot; oracle/hyq_oracle_step.c), timed on
                  this host's cores (median of 5 tokens after 2 warm-ups);
  cpu_baselines   the same restatement on every other workload (C1/C2 GEMVs,
                  a 256-row sample of each C4 GEMM, the C5 MoE layer), with the
                  host's CPU model and core count; beside them the GPU path's
                  int8 algorithm in portable C (not a reference path on x86).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0
ROOFLINE_PROFILE = "decode_attention_1p8b_ctx1153"
METRIC = "decode tok/s 1.8B Q2_0C; quant GEMV HBM GB/s as % of ~8 TB/s peak"
PREFILLED = 1024


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Events:
    """hipEvent timing on a given stream (the HIP runtime libhyq links)."""

    def __init__(self, stream: int):
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.stream = ctypes.c_void_p(stream)

    def graph_ms(self, fn, n: int, replays: int = 10) -> float:
        """Captures fn(0) .. fn(n-1) (launches on the stream) into one HIP
        graph and returns the average ms per replay of it (after one untimed
        replay): back-to-back launches with no host work between them."""
        h = self.hip
        graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
        assert h.hipStreamSynchronize(self.stream) == 0
        assert h.hipStreamBeginCapture(self.stream, 1) == 0  # thread-local mode
        for i in range(n):
            fn(i)
        assert h.hipStreamEndCapture(self.stream, ctypes.byref(graph)) == 0
        assert h.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        ms = self.time_ms(lambda i: h.hipGraphLaunch(exe, self.stream), replays)
        h.hipGraphExecDestroy(exe)
        h.hipGraphDestroy(graph)
        return ms

    def _ev(self):
        e = ctypes.c_void_p()
        assert self.hip.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def time_ms(self, fn, iters: int) -> float:
        """Average ms per call of fn(i) over iters calls (after one untimed call)."""
        s, e = self._ev(), self._ev()
        fn(0)
        self.hip.hipEventRecord(s, self.stream)
        for i in range(iters):
            fn(i)
        self.hip.hipEventRecord(e, self.stream)
        self.hip.hipEventSynchronize(e)
        ms = ctypes.c_float()
        self.hip.hipEventElapsedTime(ctypes.byref(ms), s, e)
        self.hip.hipEventDestroy(s)
        self.hip.hipEventDestroy(e)
        return ms.value / iters


ROTATE_BYTES = 1 << 30  # distinct weight copies per measurement: 4x the 256 MB MALL


def gemv_rate(hyq, ctx, ev, dtype, rows, cols, seed=1, min_bytes=ROTATE_BYTES, graph=True):
    """Standalone int8 GEMV with Q8 input over >= 1 GiB of distinct weight
    copies: (us per launch, algorithmic GB/s) from back-to-back launches, and
    the aggregate GB/s of one HIP graph that launches every copy once."""
    from synth import random_matrix
    base = random_matrix(dtype, rows, cols, seed=seed)
    copies = int(min(2048, max(2, np.ceil(min_bytes / base.size))))
    Ws = [ctx.upload(dtype, base, (cols, rows)) for _ in range(copies)]
    x = np.random.default_rng(seed).normal(0, 1, cols).astype(np.float32)
    q8 = ctx.q8(cols)
    xd = ctx.array(x)
    q8.quantize_into(xd.ptr)
    y = ctx.empty(rows, np.float32)
    L = hyq.lib()

    def launch(i):
        L.hyq_gemv_q8_d(ctx.handle, Ws[i % copies].handle, q8.handle, None, y.ptr)

    ms = ev.time_ms(launch, max(64, 2 * copies))
    gms = ev.graph_ms(launch, copies) if graph else None
    alg = base.size + cols + 4 * (cols // 256) + 4 * rows
    for W in Ws:
        W.release()
    agg = alg * copies / (gms * 1e-3) / 1e9 if gms else None
    return ms * 1e3, alg / (ms * 1e-3) / 1e9, agg, copies, alg


def gemv_silu_rate(hyq, ctx, ev, dtype, rows, cols, seed=1, min_bytes=ROTATE_BYTES):
    """The fused gate/up launch of a decode step (GEMV_SILU: gate and up
    [rows x cols] each, y = silu(gate x) * (up x), Weight::
    matmul_gate_up_silu_fast) with Q8 input, over >= 1 GiB of distinct weight
    pairs: (us per launch, algorithmic GB/s, algorithmic bytes)."""
    from synth import random_matrix
    g = random_matrix(dtype, rows, cols, seed=seed)
    u = random_matrix(dtype, rows, cols, seed=seed + 1)
    pairs = int(min(1024, max(2, np.ceil(min_bytes / (2 * g.size)))))
    Gs = [ctx.upload(dtype, g, (cols, rows)) for _ in range(pairs)]
    Us = [ctx.upload(dtype, u, (cols, rows)) for _ in range(pairs)]
    x = np.random.default_rng(seed).normal(0, 1, cols).astype(np.float32)
    q8 = ctx.q8(cols)
    xd = ctx.array(x)
    q8.quantize_into(xd.ptr)
    y = ctx.empty(rows, np.float32)
    L = hyq.lib()

    def launch(i):
        L.hyq_gate_up_silu_q8_d(ctx.handle, Gs[i % pairs].handle, Us[i % pairs].handle,
                                q8.handle, y.ptr)

    ms = ev.time_ms(launch, max(64, 2 * pairs))
    alg = 2 * g.size + cols + 4 * (cols // 256) + 4 * rows
    for W in Gs + Us:
        W.release()
    q8.release()
    return ms * 1e3, alg / (ms * 1e-3) / 1e9, alg


def decode_line(hyq, ctx, model, prefilled, warmup, steps, use_graph, seed=0) -> dict:
    """Greedy decode of a synthetic dense model: `warmup` untimed steps, then
    `steps` timed ones (hyq_dense_generate, one HIP graph replay per token,
    synchronised before it returns) from a KV cache pre-filled with N(0,1) to
    `prefilled` positions; tok/s and the HBM rate of the bytes a token
    streams (packed weights, the tied lm_head once, K/V at the mid position)."""
    from synth import dense_weight_bytes, load_dense, make_kv_cache
    cfg = model["cfg"]
    context = prefilled + warmup + steps + 1
    kv = make_kv_cache(cfg, context, prefilled, seed=seed)
    dec = load_dense(hyq, ctx, model, context)
    for l in range(cfg["layers"]):
        dec.load_kv(l, kv[0][l, :prefilled], kv[1][l, :prefilled])
    dec.position = prefilled
    toks = dec.generate(1, warmup, use_graph=use_graph) if warmup else [1]
    t0 = time.perf_counter()
    dec.generate(int(toks[-1]), steps, use_graph=use_graph)
    dt = time.perf_counter() - t0
    dec.close()
    tok_s = steps / dt
    kvw = cfg["kv_heads"] * cfg["head_dim"]
    mid = prefilled + warmup + steps // 2
    step_bytes = dense_weight_bytes(model) + cfg["layers"] * 2 * (mid + 1) * kvw * 4
    return dict(tok_s=round(tok_s, 2), ms_per_token=round(dt / steps * 1e3, 4), steps=steps,
                warmup=warmup, positions=[prefilled + warmup, prefilled + warmup + steps - 1],
                step_hbm=dict(bytes_per_token=int(step_bytes),
                              GBs=round(step_bytes * tok_s / 1e9, 1),
                              frac=round(step_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4)))


DENSE_7B = dict(layers=32, hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=14336,
                vocab=128167, rope_base=11158840.0, rms_eps=1e-5)


def stq_zero_fraction(ctx, rows, cols, seed=1, sample=64) -> float:
    """Fraction of zero weights in the first `sample` rows of the synthetic
    STQ1_0 matrix gemv_rate uploads, decoded on the device."""
    from synth import STQ1_0, random_matrix
    W = ctx.upload(STQ1_0, random_matrix(STQ1_0, rows, cols, seed=seed), (cols, rows))
    vals = np.concatenate([W.row(r) for r in range(min(sample, rows))])
    W.release()
    return round(float(np.mean(vals == 0.0)), 4)


def read_ceiling(hyq, ctx, ev, nbytes=2 << 30):
    """The read-only HBM rate: one 2 GiB buffer (8x the MALL) read once per
    launch by the streaming kernel, best over workgroup counts."""
    L = hyq.lib()
    buf = ctx.empty(nbytes, np.uint8)
    sink = ctx.empty(1 << 16, np.float32)
    best = None
    for wgs in (1024, 4096, 16384, 65536):
        ms = ev.time_ms(lambda i: L.hyq_hbm_read_d(ctx.handle, buf.ptr, nbytes, wgs, sink.ptr), 10)
        gbs = nbytes / (ms * 1e-3) / 1e9
        if best is None or gbs > best["GBs"]:
            best = dict(bytes=nbytes, workgroups=wgs, ms=round(ms, 4), GBs=round(gbs, 1))
    buf.free()
    return best


def sized_read_ceiling(hyq, ctx, ev, nbytes, pool=2 << 30) -> dict:
    """The read-only rate of one launch that reads `nbytes`: the streaming
    kernel over windows of that size rotated through a 2 GiB buffer (no
    window is read again before the other 2 GiB have been), back-to-back
    launches, best over workgroup counts - what any kernel moving that many
    bytes per launch can reach, launch and ramp included."""
    L = hyq.lib()
    n = -(-nbytes // 256) * 256
    windows = max(2, pool // n)
    buf = ctx.empty(windows * n, np.uint8)
    sink = ctx.empty(1 << 16, np.float32)
    best = None
    for wgs in (256, 512, 1024, 2048, 4096, 8192):
        ms = ev.time_ms(lambda i: L.hyq_hbm_read_d(ctx.handle, buf.ptr + (i % windows) * n, n,
                                                   wgs, sink.ptr), max(64, windows))
        gbs = n / (ms * 1e-3) / 1e9
        if best is None or gbs > best["GBs"]:
            best = dict(us=round(ms * 1e3, 3), workgroups=wgs, GBs=round(gbs, 1))
    buf.free()
    sink.free()
    return best


MFMA_F16_PEAK_TFLOPS = 2500.0
HIP_ATTR_CLOCK_KHZ, HIP_ATTR_CUS = 5, 63  # hipDeviceAttributeClockRate, ...MultiprocessorCount


def mfma_ceiling(hyq, ctx, ev, iters: int = 2048) -> dict:
    """The sustained f16 MFMA rate of this device: 8 workgroups of 4 waves per
    CU, each wave issuing back-to-back independent v_mfma_f32_32x32x16_f16 on
    register operands (hyq_mfma_stream_d), best of 5 launches - the practical
    ceiling of the batched products, as read_ceiling is of the GEMVs."""
    cu = ctypes.c_int()
    ev.hip.hipDeviceGetAttribute(ctypes.byref(cu), HIP_ATTR_CUS, 0)
    wgs = 8 * cu.value
    sink = ctx.empty(wgs * 256, np.float32)
    L = hyq.lib()
    best = None
    for _ in range(5):
        ms = ev.time_ms(lambda i: L.hyq_mfma_stream_d(ctx.handle, wgs, iters, sink.ptr), 1)
        best = ms if best is None or ms < best else best
    flop = wgs * 4.0 * iters * 4 * 32768
    return dict(workgroups=wgs, TFLOPs=round(flop / (best * 1e-3) / 1e12, 1))


def mfma_peak_from_clock(ev, device: int = 0) -> dict:
    """The dense f16 MFMA peak recomputed from the device's CU count and peak
    clock: 4 SIMDs per CU, each a 32x32x16 f16 MFMA (32,768 flop) per 32
    cycles, i.e. 4,096 flop per clock per CU."""
    cl, cu = ctypes.c_int(), ctypes.c_int()
    ev.hip.hipDeviceGetAttribute(ctypes.byref(cl), HIP_ATTR_CLOCK_KHZ, device)
    ev.hip.hipDeviceGetAttribute(ctypes.byref(cu), HIP_ATTR_CUS, device)
    tf = cu.value * 4096 * cl.value * 1e3 / 1e12
    return dict(cus=cu.value, clock_mhz=round(cl.value / 1e3, 1), TFLOPs=round(tf, 1))


def prefill_rate(hyq, ctx, ev, dtype, rows, cols, batch, seed=3):
    """Batched matmul (f16 MFMA): (us per launch, TFLOP/s) at [rows x cols] x
    [cols x batch], inputs resident in HBM."""
    from synth import random_matrix
    w = random_matrix(dtype, rows, cols, seed=seed)
    W = ctx.upload(dtype, w, (cols, rows))
    x = ctx.array(np.random.default_rng(seed).normal(0, 1, batch * cols).astype(np.float32))
    y = ctx.empty(batch * rows, np.float32)
    L = hyq.lib()

    def launch(i):
        L.hyq_matmul_d(ctx.handle, W.handle, x.ptr, batch, y.ptr)

    ms = ev.time_ms(launch, 20)
    flop = 2.0 * rows * cols * batch
    W.release()
    return ms * 1e3, flop / (ms * 1e-3) / 1e12


def prefill_e2e(dec, cfg, tokens: int, runs: int = 3) -> dict:
    """Model::prefill_into of a `tokens`-token prompt from position 0 (chunks of
    256 through the batch > 1 forward pass, last row's logits and argmax):
    best wall-clock time of `runs` after one untimed run. linear_TFLOPs counts
    2 * tokens * (Q/K/V/o/gate/up/down weights) multiply-adds per second."""
    ids = np.random.default_rng(11).integers(0, cfg["vocab"], tokens).astype(np.int32)
    best = None
    for r in range(runs + 1):
        dec.position = 0
        t0 = time.perf_counter()
        dec.prefill(ids, want_logits=False)
        dt = time.perf_counter() - t0
        if r and (best is None or dt < best):
            best = dt
    H, F, D = cfg["hidden"], cfg["ffn"], cfg["head_dim"]
    QL, KV = cfg["heads"] * D, cfg["kv_heads"] * D
    per_layer = H * (QL + 2 * KV) + QL * H + 2 * H * F + F * H
    flop = 2.0 * tokens * cfg["layers"] * per_layer
    return dict(tokens=tokens, ms=round(best * 1e3, 3), tok_s=round(tokens / best, 1),
                linear_TFLOPs=round(flop / best / 1e12, 1))


def moe_rate(hyq, ctx, ev, tokens=64, experts=64, used=8, hidden=2048, mid=1536, seed=5):
    """MoE layer at 30B-A3B-style shapes: the dense Q8_0 shared projection
    [2048x2048] seeds the output (batched matmul), then the Q4_K expert loop
    (softmax top-8 routing of N(0,1) logits, weights renormalized).
    hyq_moe_shared_experts_d runs the shared product inside the expert
    launches (`us`); `us_two_calls` times hyq_matmul_d then
    hyq_moe_experts_d."""
    from synth import Q4_K, Q8_0, random_matrix
    rng = np.random.default_rng(seed)
    G = ctx.upload(Q4_K, random_matrix(Q4_K, experts * mid, hidden, seed), (hidden, mid, experts))
    U = ctx.upload(Q4_K, random_matrix(Q4_K, experts * mid, hidden, seed + 1),
                   (hidden, mid, experts))
    D = ctx.upload(Q4_K, random_matrix(Q4_K, experts * hidden, mid, seed + 2),
                   (mid, hidden, experts))
    S = ctx.upload(Q8_0, random_matrix(Q8_0, hidden, hidden, seed + 3), (hidden, hidden))
    pt, pe, pw = [], [], []
    for t in range(tokens):
        z = rng.normal(0, 1, experts)
        p = np.exp(z - z.max())
        p /= p.sum()
        idx = sorted(range(experts), key=lambda i: (-p[i], i))[:used]
        pt += [t] * used
        pe += idx
        pw += list(p[idx] / p[idx].sum())
    x = ctx.array(rng.normal(0, 1, tokens * hidden).astype(np.float32))
    out = ctx.empty(tokens * hidden, np.float32)
    ptd = ctx.array(np.array(pt, np.int32))
    ped = ctx.array(np.array(pe, np.int32))
    pwd = ctx.array(np.array(pw, np.float32))
    L = hyq.lib()
    nbytes = L.hyq_moe_scratch_bytes(tokens, len(pt), experts, hidden, mid)
    scratch = ctx.empty(nbytes, np.uint8)

    def sequential(i):
        L.hyq_matmul_d(ctx.handle, S.handle, x.ptr, tokens, out.ptr)
        L.hyq_moe_experts_d(ctx.handle, G.handle, U.handle, D.handle, x.ptr, tokens, ptd.ptr,
                            ped.ptr, pwd.ptr, len(pt), scratch.ptr, nbytes, out.ptr)

    def layer(i):
        L.hyq_moe_shared_experts_d(ctx.handle, S.handle, G.handle, U.handle, D.handle, x.ptr,
                                   tokens, ptd.ptr, ped.ptr, pwd.ptr, len(pt), scratch.ptr,
                                   nbytes, out.ptr)

    ms_seq = ev.time_ms(sequential, 20)
    ms = ev.time_ms(layer, 20)
    touched = len(set(pe))
    wbytes = touched * (2 * mid * hidden // 256 * 144 + hidden * mid // 256 * 144) + \
        hidden * hidden // 32 * 34
    for w in (G, U, D, S):
        w.release()
    return dict(us=round(ms * 1e3, 2), us_two_calls=round(ms_seq * 1e3, 2),
                experts_touched=touched, weight_bytes=wbytes,
                GBs=round(wbytes / (ms * 1e-3) / 1e9, 1),
                frac=round(wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4))


def _upload_rotation(ctx, dtype, blobs, dims, min_bytes):
    """Device copies of the given GGUF blobs, cycled until they hold >= min_bytes."""
    out, total, i = [], 0, 0
    while total < min_bytes or i < len(blobs):
        b = blobs[i % len(blobs)]
        out.append(ctx.upload(dtype, b, dims))
        total += b.size
        i += 1
    return out


def step_kernel_table(hyq, ctx, ev, model, kv, pos):
    """Per-launch time (HIP events on the context stream) of the decode step's
    kernels launched in isolation through the C ABI, each with its operands
    rotated over more memory than the 256 MB Infinity Cache holds (1 GiB of
    weights, 64 inputs), so that they
    come from HBM as they do in the step (a token streams ~0.8 GB).

    `same_kernel` marks rows whose ABI call launches the very instantiation the
    step launches (same format, shape, input stage and preload depth); the
    others are the nearest ABI path (noted in `launch`)."""
    c = model["cfg"]
    L = hyq.lib()
    H, F, D = c["hidden"], c["ffn"], c["head_dim"]
    QL, KVW = c["heads"] * D, c["kv_heads"] * D
    lin = model["linear"]
    rng = np.random.default_rng(1)
    table = {}

    def staged_gemv(name, key, rows, cols, per_step, note, min_bytes=ROTATE_BYTES, same=True):
        blobs = [model["layers"][l][key] for l in range(c["layers"])]
        Ws = _upload_rotation(ctx, lin, blobs, (cols, rows), min_bytes)
        xs = [ctx.array(rng.normal(0, 1, cols).astype(np.float32)) for _ in range(64)]
        y = ctx.empty(rows, np.float32)
        n = len(Ws)

        def launch(i):
            L.hyq_matmul_d(ctx.handle, Ws[i % n].handle, xs[i % 64].ptr, 1, y.ptr)

        ms = ev.time_ms(launch, 2 * n)
        alg = blobs[0].size + 4 * cols + 4 * rows
        table[name] = dict(us=round(ms * 1e3, 3), bytes=int(alg), per_step=per_step,
                           GBs=round(alg / (ms * 1e-3) / 1e9, 1),
                           us_per_step=round(ms * 1e3 * per_step, 2), same_kernel=same,
                           launch=note)
        for W in Ws:
            W.release()

    staged_gemv("attn_output", "o", H, QL, c["layers"],
                "hyq_matmul_d batch 1: Q2_0C [2048 x 2048], f32 input quantized in the launch: "
                "the instantiation the step launches for the attention output (+ residual)")
    staged_gemv("down", "down", H, F, c["layers"],
                "hyq_matmul_d batch 1: Q2_0C [2048 x 6144] as one launch (the step splits it "
                "into three K slices of the attention-output kernel instead)", same=False)

    # the step's attention launch (RoPE, q/k norms, KV append, split partials)
    # and its merge, over the prefilled cache at the bench's positions, K/V
    # rotated over 64 layer caches (~150 MB)
    ctxlen = kv[0].shape[1]
    ks = [ctx.array(np.ascontiguousarray(kv[0][l % c["layers"]])) for l in range(64)]
    vs = [ctx.array(np.ascontiguousarray(kv[1][l % c["layers"]])) for l in range(64)]
    qd = ctx.array(rng.normal(0, 1, QL).astype(np.float32))
    kd = ctx.array(rng.normal(0, 1, KVW).astype(np.float32))
    vd = ctx.array(rng.normal(0, 1, KVW).astype(np.float32))
    L0 = model["layers"][0]
    qn, kn = ctx.array(L0["q_norm"]), ctx.array(L0["k_norm"])
    freq = ctx.array(np.array([np.float32(c["rope_base"]) ** np.float32(-2.0 * j / D)
                               for j in range(D // 2)], np.float32))
    posd = ctx.array(np.array([pos], np.int32))
    scratch = ctx.empty(L.hyq_attention_scratch_floats(ctxlen, c["heads"]), np.float32)
    out = ctx.empty(QL, np.float32)

    def att(i, o):
        L.hyq_attention_rope_d(ctx.handle, qd.ptr, kd.ptr, vd.ptr, qn.ptr, kn.ptr, freq.ptr,
                               posd.ptr, ctxlen, c["heads"], c["kv_heads"], D,
                               ctypes.c_float(c["rms_eps"]), 0, ks[i % 64].ptr, vs[i % 64].ptr,
                               scratch.ptr, o)

    ms = ev.time_ms(lambda i: att(i, None), 256)
    alg = attention_bytes(c, pos, ctxlen)
    table["attention"] = dict(us=round(ms * 1e3, 3), bytes=int(alg), per_step=c["layers"],
                              GBs=round(alg / (ms * 1e-3) / 1e9, 1),
                              us_per_step=round(ms * 1e3 * c["layers"], 2), same_kernel=True,
                              launch="hyq_attention_rope_d without its merge: the step's "
                                     "attention kernel (RoPE + q/k norms of the raw "
                                     "projections, KV append, split softmax partials of 16 "
                                     "heads over the cache)")
    ms2 = ev.time_ms(lambda i: att(i, out.ptr), 256)
    table["attention_and_merge"] = dict(
        us=round(ms2 * 1e3, 3), per_step=c["layers"], us_per_step=round(ms2 * 1e3 * c["layers"], 2),
        same_kernel=False, launch="hyq_attention_rope_d: the step's attention kernel and its "
                                  "split merge (two launches)")
    del ks, vs

    # lm_head: the tied Q6_K matrix (203 MB), two copies alternating
    E = [ctx.upload(model["embed_dtype"], model["embed"], (H, c["vocab"])) for _ in range(2)]
    xs = [ctx.array(rng.normal(0, 1, H).astype(np.float32)) for _ in range(2)]
    yl = ctx.empty(c["vocab"], np.float32)

    def head(i):
        L.hyq_matmul_d(ctx.handle, E[i % 2].handle, xs[i % 2].ptr, 1, yl.ptr)

    ms = ev.time_ms(head, 40)
    alg = model["embed"].size + 4 * H + 4 * c["vocab"]
    table["lm_head"] = dict(us=round(ms * 1e3, 3), bytes=int(alg), per_step=1,
                            GBs=round(alg / (ms * 1e-3) / 1e9, 1), us_per_step=round(ms * 1e3, 2),
                            same_kernel=False,
                            launch="hyq_matmul_d batch 1: Q6_K [120818 x 2048], f32 input "
                                   "quantized in the launch (the step also applies the output "
                                   "RMSNorm in it)")
    for W in E:
        W.release()
    return table


def attention_bytes(c, pos, ctxlen) -> int:
    """Algorithmic bytes of the step's attention launch at position `pos`:
    the cached K/V rows 0..pos-1 of every KV head read once, the raw q/k/v
    rows read, the new K/V row written, and the split partials written."""
    from_cache = 2 * pos * c["kv_heads"] * c["head_dim"] * 4
    qkv = (c["heads"] + 2 * c["kv_heads"]) * c["head_dim"] * 4
    append = 2 * c["kv_heads"] * c["head_dim"] * 4
    per = -(-ctxlen // 64)
    chunk = -(-per // 32) * 32
    nact = -(-(pos + 1) // chunk)
    partials = nact * c["heads"] * 132 * 4
    return from_cache + qkv + append + partials


def copy_rate(hyq, ctx, ev, nbytes=1 << 30):
    """Device-to-device copy bandwidth on the context stream (read + write
    bytes / time), the practical HBM ceiling beside the 8 TB/s peak."""
    L = hyq.lib()
    a, b = ctx.empty(nbytes, np.uint8), ctx.empty(nbytes, np.uint8)
    ms = ev.time_ms(lambda i: hyq.check(L.hyq_memcpy_d2d(ctx.handle, b.ptr, a.ptr, nbytes)), 10)
    a.free()
    b.free()
    return dict(bytes=2 * nbytes, ms=round(ms, 4), GBs=round(2 * nbytes / (ms * 1e-3) / 1e9, 1))


def roofline_loop(hyq, ctx, ev, model, kv, pos, iters):
    """The roofline kernel alone (for counter runs): the step's attention
    launch as step_kernel_table times it, then one 256 MiB device copy whose
    HBM traffic is known (the scale of the FETCH_SIZE / WRITE_SIZE counters)."""
    table = {}
    c = model["cfg"]
    L = hyq.lib()
    D = c["head_dim"]
    QL, KVW = c["heads"] * D, c["kv_heads"] * D
    rng = np.random.default_rng(1)
    ctxlen = kv[0].shape[1]
    ks = [ctx.array(np.ascontiguousarray(kv[0][l % c["layers"]])) for l in range(64)]
    vs = [ctx.array(np.ascontiguousarray(kv[1][l % c["layers"]])) for l in range(64)]
    qd = ctx.array(rng.normal(0, 1, QL).astype(np.float32))
    kd = ctx.array(rng.normal(0, 1, KVW).astype(np.float32))
    vd = ctx.array(rng.normal(0, 1, KVW).astype(np.float32))
    L0 = model["layers"][0]
    qn, kn = ctx.array(L0["q_norm"]), ctx.array(L0["k_norm"])
    freq = ctx.array(np.array([np.float32(c["rope_base"]) ** np.float32(-2.0 * j / D)
                               for j in range(D // 2)], np.float32))
    posd = ctx.array(np.array([pos], np.int32))
    scratch = ctx.empty(L.hyq_attention_scratch_floats(ctxlen, c["heads"]), np.float32)
    ms = ev.time_ms(lambda i: L.hyq_attention_rope_d(
        ctx.handle, qd.ptr, kd.ptr, vd.ptr, qn.ptr, kn.ptr, freq.ptr, posd.ptr, ctxlen,
        c["heads"], c["kv_heads"], D, ctypes.c_float(c["rms_eps"]), 0, ks[i % 64].ptr,
        vs[i % 64].ptr, scratch.ptr, None), iters)
    nb = 256 << 20
    a, b = ctx.empty(nb, np.uint8), ctx.empty(nb, np.uint8)
    hyq.check(L.hyq_memcpy_d2d(ctx.handle, b.ptr, a.ptr, nb))
    ctx.sync()
    # every buffer released here, before the context and the process end
    for d in ks + vs + [qd, kd, vd, qn, kn, freq, posd, scratch, a, b]:
        d.free()
    return ms * 1e3


def host_cpu() -> dict:
    """The host's CPU model and the cores this process may use."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return dict(model=model, nproc=len(os.sched_getaffinity(0)))


def _median_s(fn, runs: int = 5, warm: int = 2) -> float:
    """Median wall time of `runs` calls after `warm` untimed ones (the
    reference's probe warms twice, src/quant.rs:2741-2747)."""
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(runs):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return float(np.median(ts))


def cpu_baselines(model, kv) -> dict:
    """The reference's x86 path restated in C (oracle/, OpenMP over this
    host's cores; each figure the median of 5 runs after 2 warm-ups) on the
    workloads of the GPU figures: the C3 decode step, the C1/C2 GEMVs (f32
    activations: scalar Q2_0C row dot, decoded-row + AVX2 dot for the other
    formats), a bounded sample of each C4 GEMM (64-row tile decode + the
    restatement's AVX2 FMA tile GEMM, and beside it the decoded rows through
    OpenBLAS's sgemm, numpy's BLAS) and the C5 MoE layer."""
    import oracle as O
    from synth import Q2_0C, Q4_K, Q6_K, Q8_0, STQ1_0, random_matrix
    threads = O.lib().hyqo_max_threads()
    rng = np.random.default_rng(7)
    out = dict(host=host_cpu(), threads=threads, runs="median of 5 after 2 warm-ups")
    # C3: one decode token of the 1.8B 2Bit model per run (x86 arm)
    o = O.DenseOracle(model)
    k, v = kv
    pos = [PREFILLED]

    def step():
        o.step(k, v, pos[0], 5, int8_path=False)
        pos[0] = PREFILLED + (pos[0] - PREFILLED + 1) % 8
    t = _median_s(step)
    out["C3_decode"] = dict(tok_s=round(1.0 / t, 3), ms=round(t * 1e3, 2),
                            sample="1 token at positions 1024..1031 per run")

    # the int8 algorithm of the GPU path restated in portable C (Q8
    # activations, integer block sums): not a reference path on x86
    def step8():
        o.step(k, v, pos[0], 5, int8_path=True)
        pos[0] = PREFILLED + (pos[0] - PREFILLED + 1) % 8
    t8 = _median_s(step8)
    out["C3_decode_int8_algorithm"] = dict(
        tok_s=round(1.0 / t8, 3), ms=round(t8 * 1e3, 2),
        note="the GPU path's int8 algorithm in portable C; not a reference path on x86")
    # C1 / C2 GEMVs at batch 1
    gemv = {}
    for name, (dt_, rows, cols) in {
        "C1_Q4_K_6144x2048": (Q4_K, 6144, 2048),
        "C2_Q2_0C_qkv_3072x2048": (Q2_0C, 3072, 2048),
        "C2_Q2_0C_attn_out_2048x2048": (Q2_0C, 2048, 2048),
        "C2_Q2_0C_gate_up_12288x2048": (Q2_0C, 12288, 2048),
        "C2_Q2_0C_down_2048x6144": (Q2_0C, 2048, 6144),
        "C2_STQ1_0_qkv_3072x2048": (STQ1_0, 3072, 2048),
        "C2_STQ1_0_attn_out_2048x2048": (STQ1_0, 2048, 2048),
        "C2_STQ1_0_gate_up_12288x2048": (STQ1_0, 12288, 2048),
        "C2_STQ1_0_down_2048x6144": (STQ1_0, 2048, 6144),
        "C2_Q6_K_lm_head_120818x2048": (Q6_K, 120818, 2048),
    }.items():
        w = random_matrix(dt_, rows, cols, seed=1)
        x = rng.normal(0, 1, cols).astype(np.float32)
        t = _median_s(lambda: O.matmul(dt_, w, rows, cols, x, 1))
        alg = w.size + 4 * cols + 4 * rows
        gemv[name] = dict(us=round(t * 1e6, 1), GBs=round(alg / t / 1e9, 2))
    out["gemv"] = gemv
    # C4: the first 256 rows of each weight at 512 tokens
    pre = {}
    for name, (dt_, rows, cols) in {
        "C4_Q4_K_gate_up_14336x4096x512": (Q4_K, 14336, 4096),
        "C4_Q6_K_down_4096x14336x512": (Q6_K, 4096, 14336),
        "C4_Q4_K_qkv_6144x4096x512": (Q4_K, 6144, 4096),
    }.items():
        n = 256
        w = random_matrix(dt_, n, cols, seed=3)
        x = rng.normal(0, 1, 512 * cols).astype(np.float32)
        t = _median_s(lambda: O.matmul(dt_, w, n, cols, x, 512), runs=5, warm=1)
        # the same work with a BLAS GEMM (the reference's candle GEMM is a
        # tuned one): decode the rows, then OpenBLAS sgemm through numpy
        xm = x.reshape(512, cols)
        tb = _median_s(lambda: xm @ O.decode(dt_, w).reshape(n, cols).T, runs=5, warm=1)
        pre[name] = dict(GFLOPs=round(2.0 * n * cols * 512 / t / 1e9, 1),
                         GFLOPs_openblas=round(2.0 * n * cols * 512 / tb / 1e9, 1),
                         sample=f"rows 0..255 of {rows} at 512 tokens ({t * 1e3:.0f} ms; "
                                f"decode + OpenBLAS sgemm {tb * 1e3:.0f} ms)")
    out["prefill"] = pre
    # C5: the MoE layer (shared Q8_0 projection + 64 tokens x top-8 Q4_K experts)
    E, U, Hd, M, T = 64, 8, 2048, 1536, 64
    G = random_matrix(Q4_K, E * M, Hd, 5)
    Uw = random_matrix(Q4_K, E * M, Hd, 6)
    D = random_matrix(Q4_K, E * Hd, M, 7)
    S = random_matrix(Q8_0, Hd, Hd, 8)
    x = rng.normal(0, 1, T * Hd).astype(np.float32)
    pt = np.repeat(np.arange(T), U).astype(np.int32)
    pe = np.concatenate([np.sort(rng.choice(E, U, replace=False)) for _ in range(T)]).astype(
        np.int32)
    pw = np.full(T * U, 1.0 / U, np.float32)

    def moe():
        seed = O.matmul(Q8_0, S, Hd, Hd, x, T).reshape(-1)
        O.moe_experts(Q4_K, Q4_K, G, Uw, D, E, Hd, M, x, pt, pe, pw, seed)
    t = _median_s(moe, runs=5, warm=1)
    out["moe"] = dict(us=round(t * 1e6, 1),
                      sample="64 tokens, top-8 of 64 Q4_K experts (width 1536) + Q8_0 shared "
                             "[2048x2048]")
    out["headline"] = dict(
        value=out["C3_decode"]["tok_s"], unit="tok/s", cores=threads, kind="port",
        sample=f"one greedy decode token per run at positions 1024..1031, median of 5 after 2 "
               f"warm-ups, of the same synthetic 1.8B 2Bit model and KV cache: the x86 path of "
               f"Model::forward_into (f32 activations) restated in C, {threads} OpenMP threads "
               f"on {out['host']['nproc']} cores of {out['host']['model']}")
    return out


# single-kernel loops for counter runs: (kind, format, rows, cols)
ONLY = {
    "c4_q4k_gate_up_14336x4096x512": ("gemm", "Q4_K", 14336, 4096),
    "c4_q6k_down_4096x14336x512": ("gemm", "Q6_K", 4096, 14336),
    "gemv_stq1_0_gate_up_28672x4096": ("gemv", "STQ1_0", 28672, 4096),
    "gemv_q4k_gate_14336x4096": ("gemv", "Q4_K", 14336, 4096),
    "c5_moe_layer_64tok_top8of64": ("moe", None, 0, 0),
    "decode_7b_q4km": ("decode", "7B", 0, 0),
    "decode_1p8b_stq1_0": ("decode", "STQ1_0", 0, 0),
    "decode_1p8b_q2c": ("decode", "Q2_0C", 0, 0),
}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=120)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-gemv", action="store_true", help="skip the standalone GEMV table")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the batched (prefill) GEMM table")
    ap.add_argument("--no-models", action="store_true",
                    help="skip the 1.8B 1.25Bit and 7B Q4_K_M decode lines")
    ap.add_argument("--roofline-only", action="store_true",
                    help="run only the roofline kernel loop and a 256 MiB copy (for hardware "
                         "counter runs), print its time and exit")
    ap.add_argument("--only", choices=sorted(ONLY),
                    help="run only this kernel's measurement loop (for hardware counter "
                         "runs), print its time and exit")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch the step's kernels one by one instead of replaying a HIP "
                         "graph, and skip the GEMVs' graph aggregates (for profilers that "
                         "cannot follow graph capture)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the path has no multi-GPU runtime in this build)", file=sys.stderr)
        return 2
    import __graft_entry__ as ge
    from synth import DENSE_1P8B, NAMES, Q2_0C, Q4_K, Q6_K, STQ1_0, dense_weight_bytes, \
        load_dense, make_dense_model, make_kv_cache

    hyq = ge.package()
    if args.only:
        ctx = hyq.Context(0)
        ev = Events(ctx.stream)
        kind, dt_name, rows, cols = ONLY[args.only]
        dt_ = dict(Q4_K=Q4_K, Q6_K=Q6_K, STQ1_0=STQ1_0, Q2_0C=Q2_0C).get(dt_name)
        if kind == "moe":
            m = moe_rate(hyq, ctx, ev)
            print(json.dumps({"kernel": args.only, "avg_us": m["us"], "GBs": m["GBs"],
                              "two_calls_us": m["us_two_calls"]}), flush=True)
        elif kind == "decode":
            mcfg, lin, down = ((DENSE_7B, Q4_K, Q6_K) if dt_name == "7B" else
                               (DENSE_1P8B, STQ1_0 if dt_name == "STQ1_0" else Q2_0C, None))
            m = make_dense_model(mcfg, linear=lin, embed=Q6_K, seed=2, down=down)
            r = decode_line(hyq, ctx, m, PREFILLED, args.warmup, args.steps,
                            not args.no_graph, seed=2)
            print(json.dumps({"decode": args.only, **r}), flush=True)
        elif kind == "gemm":
            us, tf = prefill_rate(hyq, ctx, ev, dt_, rows, cols, 512)
            print(json.dumps({"kernel": args.only, "avg_us": round(us, 3),
                              "TFLOPs": round(tf, 1)}), flush=True)
        else:
            us, gbs, _, copies, _ = gemv_rate(hyq, ctx, ev, dt_, rows, cols, graph=False)
            print(json.dumps({"kernel": args.only, "avg_us": round(us, 3), "GBs": round(gbs, 1),
                              "copies": copies}), flush=True)
        ctx.close()
        return 0
    cfg = DENSE_1P8B
    context = PREFILLED + args.warmup + args.steps + 1
    log("building the synthetic 1.8B 2Bit model")
    model = make_dense_model(cfg, linear=Q2_0C, embed=Q6_K, seed=0)
    kv = make_kv_cache(cfg, context, PREFILLED, seed=0)

    ctx = hyq.Context(0)
    ev = Events(ctx.stream)
    if args.roofline_only:
        us = roofline_loop(hyq, ctx, ev, model, kv, PREFILLED + args.warmup,
                           max(args.steps, 64))
        ctx.close()
        assert ev.hip.hipDeviceSynchronize() == 0
        print(json.dumps({"kernel": "attention", "avg_us": round(us, 3)}), flush=True)
        return 0
    dec = load_dense(hyq, ctx, model, context)
    for l in range(cfg["layers"]):
        dec.load_kv(l, kv[0][l, :PREFILLED], kv[1][l, :PREFILLED])
    dec.position = PREFILLED
    log("decoding")
    use_graph = not args.no_graph
    toks = dec.generate(1, args.warmup, use_graph=use_graph) if args.warmup else [1]
    t0 = time.perf_counter()
    toks = dec.generate(int(toks[-1]), args.steps, use_graph=use_graph)
    dt = time.perf_counter() - t0
    tok_s = args.steps / dt
    log(f"decode: {tok_s:.1f} tok/s ({dt / args.steps * 1e3:.3f} ms/token)")

    # the step's kernels, each timed alone with HBM-resident operands
    table = step_kernel_table(hyq, ctx, ev, model, kv, PREFILLED + args.warmup)
    dom = max((n for n in table if table[n]["same_kernel"]),
              key=lambda n: table[n]["us_per_step"])
    dk = table[dom]
    achieved = dk["bytes"] / (dk["us"] * 1e-6) / 1e9
    traffic, fetch = None, None
    tf = os.path.join(ROOT, "profiles", f"{ROOFLINE_PROFILE}_traffic.json")
    if os.path.exists(tf):
        with open(tf) as f:
            rec = json.load(f)
        traffic = rec.get("bytes_per_launch")
        fetch = rec.get("fetch_bytes_per_launch")
    roofline = dict(kernel=f"{dom}: {dk['launch']}", bound="hbm", achieved=round(achieved, 1),
                    peak=HBM_PEAK_GBS, unit="GB/s", frac=round(achieved / HBM_PEAK_GBS, 4),
                    traffic=traffic, fetch_bytes=fetch, algorithmic_bytes=dk["bytes"],
                    avg_us=dk["us"])
    copy = copy_rate(hyq, ctx, ev)
    roofline["device_copy_GBs"] = copy["GBs"]
    ceiling = read_ceiling(hyq, ctx, ev)
    roofline["read_ceiling_GBs"] = ceiling["GBs"]
    log(f"HBM: device copy {copy['GBs']:.0f} GB/s, read-only stream {ceiling['GBs']:.0f} GB/s")
    # the whole step against the same peak: bytes a token streams from HBM
    kvw = cfg["kv_heads"] * cfg["head_dim"]
    mid = PREFILLED + args.warmup + args.steps // 2
    step_bytes = dense_weight_bytes(model) + cfg["layers"] * 2 * (mid + 1) * kvw * 4
    step = dict(bytes_per_token=int(step_bytes),
                GBs=round(step_bytes * tok_s / 1e9, 1),
                frac=round(step_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4))

    gemv = {}
    if not args.no_gemv:
        for name, (dt_, rows, cols) in {
            "C1_Q4_K_6144x2048": (Q4_K, 6144, 2048),
            "C2_Q2_0C_qkv_3072x2048": (Q2_0C, 3072, 2048),
            "C2_Q2_0C_attn_out_2048x2048": (Q2_0C, 2048, 2048),
            "C2_Q2_0C_gate_up_12288x2048": (Q2_0C, 12288, 2048),
            "C2_Q2_0C_down_2048x6144": (Q2_0C, 2048, 6144),
            "C2_STQ1_0_qkv_3072x2048": (STQ1_0, 3072, 2048),
            "C2_STQ1_0_attn_out_2048x2048": (STQ1_0, 2048, 2048),
            "C2_STQ1_0_gate_up_12288x2048": (STQ1_0, 12288, 2048),
            "C2_STQ1_0_down_2048x6144": (STQ1_0, 2048, 6144),
            "C2_Q6_K_lm_head_120818x2048": (Q6_K, 120818, 2048),
            # the same kernels at 7B shapes (hidden 4096, FFN 14336)
            "7B_Q4_K_qkv_6144x4096": (Q4_K, 6144, 4096),
            "7B_Q4_K_gate_14336x4096": (Q4_K, 14336, 4096),
            "7B_Q6_K_down_4096x14336": (Q6_K, 4096, 14336),
            "7B_Q2_0C_gate_up_28672x4096": (Q2_0C, 28672, 4096),
            "7B_STQ1_0_gate_up_28672x4096": (STQ1_0, 28672, 4096),
            # the target formats at the 7B vocabulary projection's shape
            # (an lm_head in that format): sizes where the HBM stream, not
            # the ~3 us launch ramp, decides
            "7B_vocab_Q4_K_128167x4096": (Q4_K, 128167, 4096),
            "7B_vocab_Q2_0C_128167x4096": (Q2_0C, 128167, 4096),
            "7B_vocab_STQ1_0_128167x4096": (STQ1_0, 128167, 4096),
        }.items():
            us, gbs, agg, copies, alg = gemv_rate(hyq, ctx, ev, dt_, rows, cols, graph=use_graph)
            ceil = sized_read_ceiling(hyq, ctx, ev, alg)
            gemv[name] = dict(us=round(us, 3), GBs=round(gbs, 1),
                              frac=round(gbs / HBM_PEAK_GBS, 4), copies=copies,
                              graph_GBs=round(agg, 1) if agg else None,
                              graph_frac=round(agg / HBM_PEAK_GBS, 4) if agg else None,
                              read_ceiling_same_bytes=ceil,
                              of_read_ceiling=round(gbs / ceil["GBs"], 4))
            if dt_ == STQ1_0:
                # the synthetic codes' zero fraction (uniform index and sign
                # bytes; every codebook entry has one zero digit), measured
                # on 64 rows decoded by the device (Weight::row)
                gemv[name]["zero_fraction"] = stq_zero_fraction(ctx, rows, cols)
            log(f"{name}: {us:.2f} us {gbs:.0f} GB/s; graph of {copies} copies "
                f"{agg or 0:.0f} GB/s; a read-only launch of the same bytes {ceil['us']:.2f} us "
                f"{ceil['GBs']:.0f} GB/s")
        # the 7B gate/up product as a decode step launches it: one fused
        # launch of both [14336 x 4096] matrices and the SiLU epilogue
        for name, dt_ in {"7B_Q4_K_gate_up_silu_2x14336x4096": Q4_K,
                          "7B_Q2_0C_gate_up_silu_2x14336x4096": Q2_0C,
                          "7B_STQ1_0_gate_up_silu_2x14336x4096": STQ1_0}.items():
            us, gbs, alg = gemv_silu_rate(hyq, ctx, ev, dt_, 14336, 4096)
            ceil = sized_read_ceiling(hyq, ctx, ev, alg)
            gemv[name] = dict(us=round(us, 3), GBs=round(gbs, 1),
                              frac=round(gbs / HBM_PEAK_GBS, 4), bytes=int(alg),
                              read_ceiling_same_bytes=ceil,
                              of_read_ceiling=round(gbs / ceil["GBs"], 4))
            log(f"{name}: {us:.2f} us {gbs:.0f} GB/s; a read-only launch of the same bytes "
                f"{ceil['us']:.2f} us {ceil['GBs']:.0f} GB/s")

    prefill = {}
    if not args.no_prefill:
        prefill["mfma_peak_from_clock"] = mfma_peak_from_clock(ev)
        prefill["mfma_ceiling"] = mfma_ceiling(hyq, ctx, ev)
        log(f"sustained f16 MFMA rate: {prefill['mfma_ceiling']['TFLOPs']:.0f} TFLOP/s")
        for name, (dt_, rows, cols) in {
            "C4_Q4_K_gate_up_14336x4096x512": (Q4_K, 14336, 4096),
            "C4_Q6_K_down_4096x14336x512": (Q6_K, 4096, 14336),
            "C4_Q4_K_qkv_6144x4096x512": (Q4_K, 6144, 4096),
        }.items():
            us, tf = prefill_rate(hyq, ctx, ev, dt_, rows, cols, 512)
            clk = prefill["mfma_peak_from_clock"]["TFLOPs"]
            ceil = prefill["mfma_ceiling"]["TFLOPs"]
            prefill[name] = dict(us=round(us, 2), TFLOPs=round(tf, 1),
                                 frac=round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                                 frac_of_clock_peak=round(tf / clk, 4) if clk else None,
                                 of_mfma_ceiling=round(tf / ceil, 4) if ceil else None)
            log(f"{name}: {us:.1f} us {tf:.0f} TFLOP/s")

    pf = None
    if not args.no_prefill:
        pf = prefill_e2e(dec, cfg, PREFILLED)
        log(f"1.8B prefill of a {PREFILLED}-token prompt: {pf['ms']:.2f} ms, "
            f"{pf['tok_s']:.0f} tok/s, {pf['linear_TFLOPs']:.0f} TFLOP/s in the linears")

    moe = None
    if not args.no_prefill:
        moe = moe_rate(hyq, ctx, ev)
        log(f"C5 MoE layer (64 tokens, top-8 of 64 Q4_K experts + Q8_0 shared): "
            f"{moe['us']:.1f} us {moe['GBs']:.0f} GB/s")

    # the other decode workloads the reference publishes CPU rates for
    # (docs/validation.md:68,72): the 1.8B 1.25Bit (STQ1_0) model and the 7B
    # Q4_K_M mix (Q4_K linears, Q6_K down and tied Q6_K embedding/lm_head)
    models = {}
    if not args.no_models:
        for name, (mcfg, lin, down, ref_tok_s) in {
            "1.8B_1.25Bit_STQ1_0": (cfg, STQ1_0, None, 99.32),
            "7B_Q4_K_M": (DENSE_7B, Q4_K, Q6_K, 2.96),
        }.items():
            log(f"building the synthetic {name} model")
            m = make_dense_model(mcfg, linear=lin, embed=Q6_K, seed=2, down=down)
            models[name] = decode_line(hyq, ctx, m, PREFILLED, args.warmup, args.steps,
                                       use_graph, seed=2)
            models[name]["config"] = dict(mcfg, linear=NAMES[lin], down=NAMES[down or lin],
                                          embed="Q6_K (tied)")
            models[name]["reference_published"] = dict(
                value=ref_tok_s, unit="tok/s",
                note="Apple M2 Pro 8 threads, real weights (docs/validation.md); not this config")
            del m
            log(f"decode {name}: {models[name]['tok_s']:.1f} tok/s "
                f"({models[name]['ms_per_token']:.3f} ms/token), "
                f"{models[name]['step_hbm']['GBs']:.0f} GB/s of a token's bytes")

    cpu, cpus = None, None
    if not args.no_cpu:
        log("cpu baselines")
        cpus = cpu_baselines(model, kv)
        cpu = cpus.pop("headline")
        log(f"cpu: {cpu['value']} tok/s on {cpu['cores']} threads")

    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "1.8B 2Bit greedy decode, batch 1, Q2_0C linears, Q6_K tied "
                               "embedding/lm_head, f32 KV cache pre-filled to 1024 positions",
                   "layers": cfg["layers"], "hidden": cfg["hidden"], "heads": cfg["heads"],
                   "kv_heads": cfg["kv_heads"], "ffn": cfg["ffn"], "vocab": cfg["vocab"],
                   "positions": [PREFILLED + args.warmup,
                                 PREFILLED + args.warmup + args.steps - 1],
                   "graph": use_graph},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_baselines": cpus,
        "step_hbm": step,
        "decode_kernels": table,
        "gemv": gemv,
        "decode_models": models,
        "prefill": prefill,
        "prefill_1p8b": pf,
        "moe": moe,
        "reference_published": {"value": 86.86, "unit": "tok/s",
                                "note": "Apple M2 Pro 8 threads, real weights, ~14-18 "
                                        "positions (docs/validation.md:70); not this config"},
    }
    print(json.dumps(out), flush=True)
    dec.close()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
