"""GPU parity of the dense decoder at the 1.8B shapes of the headline
workload (hidden 2048, FFN 6144, 16 query / 4 KV heads of dim 128, Q2_0C
linears, Q6_K embedding and output), against the oracle's Model::forward_into
(src/model.rs:374-546 batch 1, :549-616 batch n).

At these shapes the decoder runs the code a smaller model never reaches: the
down projection as three K slices of 2048 columns whose partial rows the next
stage adds (QKV input stage, attention-output epilogue, lm_head stage), and
attention over 36 splits of a 1152-position cache.

Two kinds of check, both at the decode bar of 1e-4 relative (2-norm) with
no exception. Each batch-1 product quantizes its f32 input to int8
(Q8::quantize_into, src/quant.rs:904-922); the device records the f32 values,
codes and scales of every such stage (hyq_ctx_set_q8_trace), and
tests/q8_proof.py shows that the codes are the quantizer's on the device's
own input, that input within 1e-4 of the oracle's (so a code where the two
differ is a rounding-midpoint flip), then runs the oracle on the device's
codes:
  * layer by layer, teacher-forced: the decoder records the hidden row after
    every layer (hyq_dense_set_trace); the oracle runs each layer on the
    GPU's own input row, KV cache and codes; the layer's output row and its
    K/V rows must agree within 1e-4, and so must the logits of the GPU's
    final row;
  * free-running: the oracle's own chain (its own hidden rows and KV cache)
    with the device's codes, step after step: the logits within 1e-4 and the
    same greedy token where the top-2 gap is clear.
Without the code substitution a single flip (about 6e-4 of a product) would
grow through the later layers of a random-init model; with it the chains
differ only by f32 rounding."""
import numpy as np
import pytest

import q8_proof as P
from synth import (DENSE_1P8B, Q2_0C, Q4_K, Q6_K, load_dense, make_dense_model, make_kv_cache,
                   random_matrix)

pytestmark = pytest.mark.gpu

C3_SHAPES = dict(DENSE_1P8B, layers=3, vocab=8192)
TRACE_BYTES = 4 << 20


def _print(*a):
    print(*a, flush=True)


def _decoder(hyq, ctx, cfg, context, prefilled, seed, untied=True):
    model = make_dense_model(cfg, linear=Q2_0C, seed=seed)
    if untied:
        model["output"] = random_matrix(Q6_K, cfg["vocab"], cfg["hidden"], seed + 50)
    dec = load_dense(hyq, ctx, model, context)
    k, v = make_kv_cache(cfg, context, prefilled, seed=seed)
    for l in range(cfg["layers"]):
        dec.load_kv(l, k[l, :prefilled], v[l, :prefilled])
    dec.position = prefilled
    return model, dec, k, v


def _teacher_forced_step(ref, dec, stages, final, cfg, pos, logits, label):
    """Each traced layer against the oracle's layer on the GPU's input row,
    cache and int8 codes; then the output norm and lm_head of the GPU's final
    row. Every flipped code explained, every output within 1e-4."""
    tr = dec.trace(1)[:, 0]
    errs, flips = [], []
    for l in range(cfg["layers"]):
        kc, vc = dec.read_kv(l, pos + 1)
        kref = np.zeros((pos + 1, kc.shape[1]), np.float32)
        vref = kref.copy()
        kref[:pos] = kc[:pos]
        vref[:pos] = vc[:pos]
        out, tap = ref.layer_tap(l, tr[l], kref, vref, pos, use=stages[l])
        errs.append(P.prove((label, l), [(tr[l + 1], out), (kc[pos], kref[pos]),
                                         (vc[pos], vref[pos])], tap, stages[l], flips))
    lg, tap = ref.output_tap(tr[-1], use=final)
    errs.append(P.prove((label, "output"), [(logits, lg)], tap, final, flips))
    _print(label, "per-layer rel on the GPU's codes (last: logits)",
           ["%.1e" % e for e in errs])
    P.print_flips(label, flips)
    return errs


def _free_running(ref, model, cfg, kf, vf, pos, token, stages, final, logits, nxt, label):
    """The oracle's own chain for this token (caches kf/vf) with the GPU's
    codes: logits within 1e-4, the same greedy token where the top-2 gap is
    clear."""
    flips = []
    ref_logits = P.step_with_device_codes(ref, cfg, P.embed_row(model, cfg, token), kf, vf,
                                          pos, stages, final, label, flips)
    rel = P.rel(logits, ref_logits)
    _print(f"{label}: free-running logits rel {rel:.2e} on the GPU's codes "
           f"({len(flips)} flipped codes explained)")
    assert rel <= P.DECODE_BAR, (label, rel)
    top = np.sort(ref_logits)[-2:]
    if top[1] - top[0] > 1e-3 * np.abs(ref_logits).max():
        assert nxt == int(np.argmax(ref_logits)), label


def test_c3_shapes_layers_match_oracle(gpu_ctx, hyq, oracle):
    """Three layers at the 1.8B shapes, cache pre-filled to 1030 of 1152
    positions; four tokens, each checked layer by layer, then the
    free-running chain."""
    cfg = C3_SHAPES
    context, prefilled, steps = 1152, 1030, 4
    model, dec, k, v = _decoder(hyq, gpu_ctx, cfg, context, prefilled, seed=7)
    ref = oracle.DenseOracle(model)
    dec.set_trace(1)
    gpu_ctx.set_q8_trace(TRACE_BYTES)
    token = 17
    for i in range(steps):
        pos = prefilled + i
        gpu_ctx.clear_q8_trace()
        logits, nxt = dec.forward(token)
        stages, final = P.split_step_records(gpu_ctx.q8_trace(), ref, cfg["layers"])
        _teacher_forced_step(ref, dec, stages, final, cfg, pos, logits, f"step {i}")
        _free_running(ref, model, cfg, k, v, pos, token, stages, final, logits, nxt,
                      f"step {i}")
        token = nxt
    gpu_ctx.set_q8_trace(None)
    dec.set_trace(None)
    dec.close()


def test_c3_full_model_matches_oracle(gpu_ctx, hyq, oracle):
    """The whole 1.8B 2Bit workload: 32 layers, vocab 120818 (tied Q6_K
    embedding/output), cache pre-filled to 1024 positions. The first token
    is checked layer by layer; four tokens free-running on the GPU's codes.
    Then the captured-graph decode loop the benchmark times must produce the
    same tokens as those eager steps."""
    cfg = DENSE_1P8B
    context, prefilled = 1152, 1024
    _print("building the 32-layer model")
    model, dec, k, v = _decoder(hyq, gpu_ctx, cfg, context, prefilled, seed=1, untied=False)
    ref = oracle.DenseOracle(model)
    dec.set_trace(1)
    gpu_ctx.set_q8_trace(TRACE_BYTES)
    token, toks = 5, []
    k0, v0 = k.copy(), v.copy()
    for i in range(4):
        pos = prefilled + i
        _print("full model step", i)
        gpu_ctx.clear_q8_trace()
        logits, nxt = dec.forward(token)
        stages, final = P.split_step_records(gpu_ctx.q8_trace(), ref, cfg["layers"])
        if i == 0:
            _teacher_forced_step(ref, dec, stages, final, cfg, pos, logits, "full step 0")
        _free_running(ref, model, cfg, k, v, pos, token, stages, final, logits, nxt,
                      f"full step {i}")
        toks.append(nxt)
        token = nxt
    gpu_ctx.set_q8_trace(None)
    dec.set_trace(None)
    # the graph loop from the same start
    for l in range(cfg["layers"]):
        dec.load_kv(l, k0[l, :prefilled], v0[l, :prefilled])
    dec.position = prefilled
    got = dec.generate(5, 4, use_graph=True)
    assert list(got) == toks, (list(got), toks)
    dec.close()


SHAPES_7B = dict(layers=2, hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=14336,
                 vocab=4096, rope_base=11158840.0, rms_eps=1e-5)


def test_7b_shapes_layers_match_oracle(gpu_ctx, hyq, oracle):
    """Two layers at the 7B Q4_K_M shapes (hidden 4096, 32/8 heads of 128,
    FFN 14336; Q4_K linears, Q6_K down and output): the down projection runs
    as four K slices of 14 groups, and the next layer's QKV input stage adds
    their partial rows over 16 groups (the two-pass register stage); the
    gate/up pair has two groups per lane. Cache pre-filled to 80 of 96
    positions; three tokens, each layer by layer and free-running, on the
    GPU's codes (1e-4)."""
    cfg = SHAPES_7B
    context, prefilled = 96, 80
    model = make_dense_model(cfg, linear=Q4_K, embed=Q6_K, seed=3, down=Q6_K)
    model["output"] = random_matrix(Q6_K, cfg["vocab"], cfg["hidden"], 53)
    dec = load_dense(hyq, gpu_ctx, model, context)
    k, v = make_kv_cache(cfg, context, prefilled, seed=3)
    for l in range(cfg["layers"]):
        dec.load_kv(l, k[l, :prefilled], v[l, :prefilled])
    dec.position = prefilled
    ref = oracle.DenseOracle(model)
    dec.set_trace(1)
    gpu_ctx.set_q8_trace(TRACE_BYTES)
    token = 9
    for i in range(3):
        pos = prefilled + i
        gpu_ctx.clear_q8_trace()
        logits, nxt = dec.forward(token)
        stages, final = P.split_step_records(gpu_ctx.q8_trace(), ref, cfg["layers"])
        _teacher_forced_step(ref, dec, stages, final, cfg, pos, logits, f"7b step {i}")
        _free_running(ref, model, cfg, k, v, pos, token, stages, final, logits, nxt,
                      f"7b step {i}")
        token = nxt
    gpu_ctx.set_q8_trace(None)
    dec.set_trace(None)
    dec.close()


@pytest.mark.parametrize("n", [300])
def test_c3_shapes_prefill_layers_match_oracle(gpu_ctx, hyq, oracle, n):
    """hyq_dense_prefill of a 300-token prompt at the 1.8B shapes after 100
    cached positions: every layer's rows against the oracle's batch-n layer
    (f32 products) on the GPU's input rows and cache, at the f16-MFMA bar;
    the last row's logits against the oracle's output matmul on the GPU's
    final row at the decode bar (the logits are a batch-1 product)."""
    cfg = C3_SHAPES
    context, prefilled = 1152, 100
    model, dec, k, v = _decoder(hyq, gpu_ctx, cfg, context, prefilled, seed=8)
    ref = oracle.DenseOracle(model)
    dec.set_trace(n)
    gpu_ctx.set_q8_trace(TRACE_BYTES)
    toks = np.random.default_rng(n).integers(0, cfg["vocab"], n).astype(np.int32)
    logits, nxt = dec.prefill(toks)
    recs = gpu_ctx.q8_trace()
    gpu_ctx.set_q8_trace(None)
    tr = dec.trace(n)
    errs = []
    for l in range(cfg["layers"]):
        kc, vc = dec.read_kv(l, prefilled + n)
        kref = np.zeros((prefilled + n, kc.shape[1]), np.float32)
        vref = kref.copy()
        kref[:prefilled] = kc[:prefilled]
        vref[:prefilled] = vc[:prefilled]
        out = ref.prefill_layer(l, tr[l], kref, vref, prefilled).reshape(n, -1)
        errs.append(P.rel(tr[l + 1], out))
        assert P.rel(kc[prefilled:], kref[prefilled:]) <= 2e-3, (l, "K rows")
        assert P.rel(vc[prefilled:], vref[prefilled:]) <= 2e-3, (l, "V rows")
    # the logits: one batch-1 product of the GPU's own final row, its int8
    # codes recorded (the pass's only Q8 stage) and any flip explained
    assert len(recs) == 1, len(recs)
    final = {0: recs[0]}
    flips = []
    lg, tap = ref.output_tap(tr[-1, -1], use=final)
    lerr = P.prove("prefill output", [(logits, lg)], tap, final, flips)
    _print("prefill per-layer rel", ["%.1e" % e for e in errs], "logits %.1e" % lerr)
    P.print_flips("prefill output", flips)
    assert max(errs) <= 2e-3, errs
    dec.set_trace(None)
    dec.close()
