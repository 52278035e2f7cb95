"""GPU parity of the dense decoder at the 1.8B shapes of the headline
workload (hidden 2048, FFN 6144, 16 query / 4 KV heads of dim 128, Q2_0C
linears, Q6_K embedding and output), against the oracle's Model::forward_into
(src/model.rs:374-546 batch 1, :549-616 batch n).

At these shapes the decoder runs the code a smaller model never reaches: the
down projection as three K slices of 2048 columns whose partial rows the next
stage adds (QKV input stage, attention-output epilogue, lm_head stage), and
attention over 36 splits of a 1152-position cache.

Two kinds of check:
  * layer by layer, teacher-forced: the decoder records the hidden row after
    every layer (hyq_dense_set_trace); the oracle runs each layer on the
    GPU's own input row and KV cache, and the layer's output must agree. The
    bars: 1e-4 relative (2-norm) for a batch-1 layer, 2e-3 for a prefill
    layer (f16 operands), and the logits of the GPU's final row at 1e-4.
  * free-running: whole steps against the oracle's own chain.

Why the free-running bar is looser. Each int8 product quantizes its f32
input (Q8::quantize_into, src/quant.rs:904-922); a last-bit difference in an
input that sits at a rounding midpoint moves one int8 code by one, which
changes that product by s * W[:, j] (s = max|x| / 127): about
max|x| / (127 |x|) of the product's norm, ~6e-4 for a Gaussian row of 2048.
Such a flip is rare per layer (the teacher-forced layers agree to ~1e-7
otherwise), but a disturbance of a hidden row grows through the later layers
of a random-init model (it causes further flips downstream): the 3-layer
chain is held to 5e-3, the 32-layer one to twice the oracle's own
sensitivity, and both to the same greedy token where the oracle's top-2 gap
is clear."""
import numpy as np
import pytest

from synth import (DENSE_1P8B, Q2_0C, Q6_K, load_dense, make_dense_model, make_kv_cache,
                   random_matrix)

pytestmark = pytest.mark.gpu

C3_SHAPES = dict(DENSE_1P8B, layers=3, vocab=8192)


def _print(*a):
    print(*a, flush=True)


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


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


def _teacher_forced_step(oracle, ref, dec, cfg, pos, logits, label):
    """Each traced layer against the oracle's layer on the GPU's input row
    and cache. Bars: 1e-4 relative for the layer's hidden row and its K/V
    rows, except where a Q8 rounding flip (see the module docstring) moved
    one code: such a layer stays within 2e-3, and at most a quarter of the
    layers may need that allowance (the inputs are seeded, the kernels
    deterministic, so the count is fixed for a given case)."""
    tr = dec.trace(1)[:, 0]
    errs = []
    for l in range(cfg["layers"]):
        kc, vc = dec.read_kv(l, pos + 1)
        kref = np.zeros((pos + 1, kc.shape[1]), np.float32)
        vref = kref.copy()
        kref[:pos] = kc[:pos]
        vref[:pos] = vc[:pos]
        out = ref.layer(l, tr[l], kref, vref, pos, int8_path=True)
        errs.append(max(_rel(tr[l + 1], out), _rel(kc[pos], kref[pos]),
                        _rel(vc[pos], vref[pos])))
    # the output norm and lm_head product of the GPU's final row: one more
    # quantized product, under the same rule
    errs.append(_rel(logits, ref.output(tr[-1], int8_path=True)))
    flips = [l for l, e in enumerate(errs) if e > 1e-4]
    _print(label, "per-layer rel (last: logits)", ["%.1e" % e for e in errs],
           "past 1e-4:", flips)
    assert max(errs) <= 2e-3, (label, errs)
    assert len(flips) <= max(1, len(errs) // 4), (label, flips)
    return errs


def test_c3_shapes_layers_match_oracle(gpu_ctx, hyq, oracle):
    """Three layers at the 1.8B shapes, cache pre-filled to 1030 of 1152
    positions; four tokens, each checked layer by layer, then the
    free-running chain."""
    cfg = C3_SHAPES
    context, prefilled, steps = 1152, 1030, 4
    model, dec, k, v = _decoder(hyq, gpu_ctx, cfg, context, prefilled, seed=7)
    ref = oracle.DenseOracle(model)
    dec.set_trace(1)
    token = 17
    for i in range(steps):
        pos = prefilled + i
        logits, nxt = dec.forward(token)
        _teacher_forced_step(oracle, ref, dec, cfg, pos, logits, f"step {i}")
        ref_logits = ref.step(k, v, pos, token, int8_path=True)
        rel = _rel(logits, ref_logits)
        _print(f"step {i}: free-running logits rel {rel:.2e}")
        assert rel <= 5e-3, (i, rel)
        top = np.sort(ref_logits)[-2:]
        if top[1] - top[0] > 1e-3 * np.abs(ref_logits).max():
            assert nxt == int(np.argmax(ref_logits))
        token = nxt
    dec.set_trace(None)
    dec.close()


def _oracle_sensitivity(oracle, ref, model, cfg, k, v, pos, token, rel=1e-4, seed=0):
    """How far the oracle's own logits move when its embedding row is
    perturbed by `rel` (relative 2-norm, seeded direction): the size of the
    disturbance one Q8 rounding flip makes in a hidden row."""
    rb = model["embed"].size // cfg["vocab"]
    h0 = oracle.decode(model["embed_dtype"], model["embed"][token * rb:(token + 1) * rb])
    d = np.random.default_rng(seed).normal(0, 1, h0.size).astype(np.float32)
    outs = []
    for h in (h0, (h0 + d * np.float32(rel * np.linalg.norm(h0) / np.linalg.norm(d)))):
        kk, vv = k.copy(), v.copy()
        h = h.astype(np.float32)
        for l in range(cfg["layers"]):
            h = ref.layer(l, h, kk[l], vv[l], pos, int8_path=True)
        outs.append(ref.output(h, int8_path=True))
    return _rel(outs[1], outs[0])


def test_c3_full_model_matches_oracle(gpu_ctx, hyq, oracle):
    """The whole 1.8B 2Bit workload: 32 layers, vocab 120818 (tied Q6_K
    embedding/output), cache pre-filled to 1024 positions. The first token
    is checked layer by layer at the decode bar. Free-running, a random-init
    model of this depth amplifies any disturbance: the oracle's own logits
    move by ~3e-2 when its embedding row is perturbed by 1e-4, the size of
    what one Q8 rounding flip does to a hidden row. The free-running steps are
    therefore held to twice that self-sensitivity (measured here, on this
    model) and to the same greedy token where the top-2 gap is clear. Then the
    captured-graph decode loop the benchmark times must produce the same
    tokens as those eager steps."""
    cfg = DENSE_1P8B
    context, prefilled = 1152, 1024
    _print("building the 32-layer model")
    model, dec, k, v = _decoder(hyq, gpu_ctx, cfg, context, prefilled, seed=1, untied=False)
    ref = oracle.DenseOracle(model)
    sens = _oracle_sensitivity(oracle, ref, model, cfg, k, v, prefilled, 5)
    _print(f"oracle self-sensitivity to a 1e-4 disturbance: {sens:.2e}")
    bar = max(5e-3, 2 * sens)
    dec.set_trace(1)
    token, toks = 5, []
    k0, v0 = k.copy(), v.copy()
    for i in range(4):
        pos = prefilled + i
        _print("full model step", i)
        logits, nxt = dec.forward(token)
        if i == 0:
            _teacher_forced_step(oracle, ref, dec, cfg, pos, logits, "full step 0")
            dec.set_trace(None)
        ref_logits = ref.step(k, v, pos, token, int8_path=True)
        rel = _rel(logits, ref_logits)
        _print(f"full model step {i}: logits rel {rel:.2e} (bar {bar:.2e})")
        assert rel <= bar, (i, rel, bar)
        top = np.sort(ref_logits)[-2:]
        if top[1] - top[0] > 1e-3 * np.abs(ref_logits).max():
            assert nxt == int(np.argmax(ref_logits))
        toks.append(nxt)
        token = nxt
    # the graph loop from the same start
    for l in range(cfg["layers"]):
        dec.load_kv(l, k0[l, :prefilled], v0[l, :prefilled])
    dec.position = prefilled
    got = dec.generate(5, 4, use_graph=True)
    assert list(got) == toks, (list(got), toks)
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
    toks = np.random.default_rng(n).integers(0, cfg["vocab"], n).astype(np.int32)
    logits, nxt = dec.prefill(toks)
    tr = dec.trace(n)
    errs = []
    for l in range(cfg["layers"]):
        kc, vc = dec.read_kv(l, prefilled + n)
        kref = np.zeros((prefilled + n, kc.shape[1]), np.float32)
        vref = kref.copy()
        kref[:prefilled] = kc[:prefilled]
        vref[:prefilled] = vc[:prefilled]
        out = ref.prefill_layer(l, tr[l], kref, vref, prefilled).reshape(n, -1)
        errs.append(_rel(tr[l + 1], out))
        assert _rel(kc[prefilled:], kref[prefilled:]) <= 2e-3, (l, "K rows")
        assert _rel(vc[prefilled:], vref[prefilled:]) <= 2e-3, (l, "V rows")
    lerr = _rel(logits, ref.output(tr[-1, -1], int8_path=True))
    _print("prefill per-layer rel", ["%.1e" % e for e in errs], "logits %.1e" % lerr)
    assert max(errs) <= 2e-3, errs
    # one quantized product of the GPU's own final row: ~1e-6 unless a Q8
    # rounding flip moved one code (then up to ~6e-4)
    assert lerr <= 2e-3, lerr
    dec.set_trace(None)
    dec.close()
