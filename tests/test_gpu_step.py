"""GPU parity of the decode-step glue and the dense batch-1 decoder against
the oracle (oracle/hyq_oracle_step.c), through the C ABI.

Tolerances (floating point; stated per test): element-wise ops within a few
f32 ulps of the oracle (the GPU's sum order and sinf/cosf/expf differ from
glibc's by an ulp); the whole step within 1e-4 relative 2-norm of the
oracle's int8 path run on the GPU's own int8 codes, each code where the two
differ shown to be a rounding-midpoint flip (tests/q8_proof.py)."""
import ctypes

import numpy as np
import pytest

import q8_proof as P
from gpu_util import device_bytes
from synth import (Q2_0C, Q6_K, STQ1_0, load_dense, make_dense_model, make_kv_cache,
                   random_matrix)

pytestmark = pytest.mark.gpu


def _print(*a):
    print(*a, flush=True)


def _f(x):
    return ctypes.c_float(x)


def test_rms_norm_q8(gpu_ctx, hyq, oracle):
    L = hyq.lib()
    for n in (2048, 6144, 512):
        rng = np.random.default_rng(n)
        x = (rng.normal(0, 3, n)).astype(np.float32)
        w = rng.normal(1, 0.02, n).astype(np.float32)
        xd, wd, yd = gpu_ctx.array(x), gpu_ctx.array(w), gpu_ctx.empty(n, np.float32)
        q8 = gpu_ctx.q8(n)
        hyq.check(L.hyq_rms_norm_q8_d(gpu_ctx.handle, xd.ptr, wd.ptr, n, _f(1e-5), yd.ptr,
                                      q8.handle))
        y = yd.numpy()
        y_ref = np.empty(n, np.float32)
        oracle.lib().hyqo_rms_norm_into(x.ctypes.data, w.ctypes.data, n, _f(1e-5),
                                        y_ref.ctypes.data, 1)
        assert np.allclose(y, y_ref, rtol=4e-7, atol=0), n
        q = device_bytes(hyq, gpu_ctx, q8.values_ptr, n).view(np.int8)
        q_ref, _ = oracle.q8_quantize(y)  # the GPU's own f32 row, quantized by the oracle
        assert np.array_equal(q, q_ref), n


def _rope_ref(oracle, x, heads, pos, base, norm, eps):
    c = np.empty(64, np.float32)
    s = np.empty(64, np.float32)
    L = oracle.lib()
    L.hyqo_rope_tables(128, _f(base), pos, c.ctypes.data, s.ctypes.data)
    x = x.copy()
    L.hyqo_rope(x.ctypes.data, heads, 128, c.ctypes.data, s.ctypes.data)
    L.hyqo_rms_norm_rows(x.ctypes.data, norm.ctypes.data, x.size, 128, _f(eps), 1)
    return x


@pytest.mark.parametrize("pos", [0, 1, 1023, 1151])
def test_rope_norm_append(gpu_ctx, hyq, oracle, pos):
    heads, kvh, D, ctxlen = 16, 4, 128, 1152
    base, eps = 11158840.0, 1e-5
    rng = np.random.default_rng(pos)
    q = rng.normal(0, 1, heads * D).astype(np.float32)
    k = rng.normal(0, 1, kvh * D).astype(np.float32)
    v = rng.normal(0, 1, kvh * D).astype(np.float32)
    qn = rng.normal(1, 0.02, D).astype(np.float32)
    kn = rng.normal(1, 0.02, D).astype(np.float32)
    freq = np.array([np.float32(base) ** np.float32(-2.0 * j / D) for j in range(64)],
                    np.float32)
    d = {n: gpu_ctx.array(a) for n, a in dict(q=q, k=k, v=v, qn=qn, kn=kn, freq=freq,
                                               pos=np.array([pos], np.int32)).items()}
    kc = gpu_ctx.array(np.zeros((ctxlen, kvh * D), np.float32))
    vc = gpu_ctx.array(np.zeros((ctxlen, kvh * D), np.float32))
    hyq.check(hyq.lib().hyq_rope_norm_append_d(
        gpu_ctx.handle, d["q"].ptr, d["k"].ptr, d["v"].ptr, d["qn"].ptr, d["kn"].ptr,
        d["freq"].ptr, d["pos"].ptr, heads, kvh, D, _f(eps), kc.ptr, vc.ptr))
    q_ref = _rope_ref(oracle, q, heads, pos, base, qn, eps)
    k_ref = _rope_ref(oracle, k, kvh, pos, base, kn, eps)
    assert np.allclose(d["q"].numpy(), q_ref, rtol=2e-5, atol=2e-6)
    kcache, vcache = kc.numpy(), vc.numpy()
    assert np.allclose(kcache[pos], k_ref, rtol=2e-5, atol=2e-6)
    assert np.array_equal(vcache[pos], v)
    others = np.delete(np.arange(ctxlen), pos)
    assert not kcache[others].any() and not vcache[others].any()


@pytest.mark.parametrize("pos", [0, 30, 31, 32, 33, 100, 1151])
def test_attention(gpu_ctx, hyq, oracle, pos):
    heads, kvh, D, ctxlen = 16, 4, 128, 1152
    rng = np.random.default_rng(pos + 1)
    q = rng.normal(0, 1, heads * D).astype(np.float32)
    kc = rng.normal(0, 1, (ctxlen, kvh * D)).astype(np.float32)
    vc = rng.normal(0, 1, (ctxlen, kvh * D)).astype(np.float32)
    qd, kd, vd = gpu_ctx.array(q), gpu_ctx.array(kc), gpu_ctx.array(vc)
    posd = gpu_ctx.array(np.array([pos], np.int32))
    scratch = gpu_ctx.empty(hyq.lib().hyq_attention_scratch_floats(ctxlen, heads), np.float32)
    out = gpu_ctx.empty(heads * D, np.float32)
    q8 = gpu_ctx.q8(heads * D)
    hyq.check(hyq.lib().hyq_attention_d(gpu_ctx.handle, qd.ptr, kd.ptr, vd.ptr, posd.ptr,
                                        ctxlen, heads, kvh, D, scratch.ptr, out.ptr, q8.handle))
    got = out.numpy()
    ref = np.empty(heads * D, np.float32)
    oracle.lib().hyqo_attention(q.ctypes.data, kc.ctypes.data, vc.ctypes.data, heads, kvh, D,
                                pos + 1, ref.ctypes.data)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6), np.abs(got - ref).max()
    qv = device_bytes(hyq, gpu_ctx, q8.values_ptr, heads * D).view(np.int8)
    assert np.array_equal(qv, oracle.q8_quantize(got)[0])


def test_causal_attention_closed_form(gpu_ctx, hyq):
    """src/model.rs:1108-1125: zero queries average the visible values."""
    heads, kvh, D, ctxlen = 2, 1, 128, 2
    vc = np.zeros((ctxlen, D), np.float32)
    vc[0, :2] = [2.0, 4.0]
    vc[1, :2] = [100.0, 200.0]
    L = hyq.lib()
    kd, vd = gpu_ctx.array(np.zeros((ctxlen, D), np.float32)), gpu_ctx.array(vc)
    qd = gpu_ctx.array(np.zeros(heads * D, np.float32))
    scratch = gpu_ctx.empty(L.hyq_attention_scratch_floats(ctxlen, heads), np.float32)
    for pos, exp in ((0, [2.0, 4.0]), (1, [51.0, 102.0])):
        out = gpu_ctx.empty(heads * D, np.float32)
        posd = gpu_ctx.array(np.array([pos], np.int32))
        hyq.check(L.hyq_attention_d(gpu_ctx.handle, qd.ptr, kd.ptr, vd.ptr, posd.ptr, ctxlen,
                                    heads, kvh, D, scratch.ptr, out.ptr, None))
        o = out.numpy().reshape(heads, D)
        assert np.array_equal(o[:, :2], np.array([exp, exp], np.float32))


def test_argmax_first_maximum_wins(gpu_ctx, hyq, oracle):
    """Greedy sampling (src/generation.rs:281-290): the first maximum wins, a
    NaN is never taken and a NaN at index 0 keeps token 0; the oracle
    restates that loop."""
    L = hyq.lib()
    rng = np.random.default_rng(0)
    cases = [rng.normal(0, 1, 120818).astype(np.float32), np.zeros(1000, np.float32),
             np.full(7, -np.inf, np.float32), np.full(5000, np.nan, np.float32)]
    x = rng.normal(0, 1, 50000).astype(np.float32)
    x[[123, 4567, 40000]] = 9.0
    cases.append(x)
    x = rng.normal(0, 1, 70000).astype(np.float32)
    x[0] = np.nan
    x[60000] = 50.0  # a larger value after a NaN at index 0 is not taken
    cases.append(x)
    x = rng.normal(0, 1, 70000).astype(np.float32)
    x[[5, 33333, 69999]] = np.nan
    x[44444] = np.inf  # +inf is a value like any other
    cases.append(x)
    x = np.full(9000, -np.inf, np.float32)
    x[[100, 8000]] = np.nan
    x[4000] = -1.0
    cases.append(x)
    for x in cases:
        xd = gpu_ctx.array(x)
        scratch = gpu_ctx.empty(128, np.float32)
        tok = gpu_ctx.empty(1, np.int32)
        hyq.check(L.hyq_argmax_d(gpu_ctx.handle, xd.ptr, x.size, scratch.ptr, tok.ptr))
        got = int(tok.numpy()[0])
        exp = oracle.lib().hyqo_argmax(x.ctypes.data, x.size)
        assert got == exp, (got, exp)


def test_embed_row(gpu_ctx, hyq, oracle):
    rows, cols = 300, 2048
    w = random_matrix(Q6_K, rows, cols, seed=3)
    W = gpu_ctx.upload(Q6_K, w, (cols, rows))
    out = gpu_ctx.empty(cols, np.float32)
    rb = w.size // rows
    # (rows: an id one past the table, which the device clamps to the last row)
    for tok, src in ((0, 0), (151, 151), (rows - 1, rows - 1), (rows, rows - 1)):
        td = gpu_ctx.array(np.array([tok], np.int32))
        hyq.check(hyq.lib().hyq_embed_row_d(gpu_ctx.handle, W.handle, td.ptr, out.ptr))
        ref = oracle.decode(Q6_K, w[src * rb:(src + 1) * rb])
        assert np.array_equal(out.numpy().view(np.uint32), ref.view(np.uint32))


# ---- the whole step ----

SMALL = dict(layers=2, hidden=512, heads=4, kv_heads=1, head_dim=128, ffn=1024, vocab=3000,
             rope_base=11158840.0, rms_eps=1e-5)


def _untied(model, seed):
    """A separate output matrix, so that argmax is not the input token's row."""
    c = model["cfg"]
    model["output"] = random_matrix(Q6_K, c["vocab"], c["hidden"], seed)
    return model


@pytest.mark.parametrize("linear", [Q2_0C, STQ1_0])
def test_dense_decoder_matches_oracle(gpu_ctx, hyq, oracle, linear):
    c = SMALL
    context, prefilled, steps = 48, 37, 6
    model = _untied(make_dense_model(c, linear=linear, seed=5), seed=55)
    dec = load_dense(hyq, gpu_ctx, model, context)
    k, v = make_kv_cache(c, context, prefilled, seed=5)
    for l in range(c["layers"]):
        dec.load_kv(l, k[l, :prefilled], v[l, :prefilled])
    dec.position = prefilled
    ref = oracle.DenseOracle(model)
    gpu_ctx.set_q8_trace(1 << 20)
    token = 11
    for i in range(steps):
        _print("step", i)
        gpu_ctx.clear_q8_trace()
        logits, nxt = dec.forward(token)
        # the oracle's own chain on the GPU's int8 codes (tests/q8_proof.py)
        P.check_step(gpu_ctx, ref, model, c, k, v, prefilled + i, token, logits, nxt,
                     f"step {i}")
        assert nxt == int(np.argmax(logits))
        token = nxt
    gpu_ctx.set_q8_trace(None)
    assert dec.position == prefilled + steps


def test_graph_replays_equal_eager_launches(gpu_ctx, hyq):
    c = SMALL
    context, prefilled, steps = 64, 20, 12
    model = make_dense_model(c, linear=Q2_0C, seed=9)
    k, v = make_kv_cache(c, context, prefilled, seed=9)
    runs = []
    for use_graph in (False, True, True):
        dec = load_dense(hyq, gpu_ctx, model, context)
        for l in range(c["layers"]):
            dec.load_kv(l, k[l, :prefilled], v[l, :prefilled])
        dec.position = prefilled
        toks = dec.generate(3, steps, use_graph=use_graph)
        logits, nxt = dec.forward(int(toks[-1]))  # eager step after the replays
        runs.append((toks, logits, nxt))
        dec.close()
    for toks, logits, nxt in runs[1:]:
        assert np.array_equal(toks, runs[0][0])
        assert np.array_equal(logits.view(np.uint32), runs[0][1].view(np.uint32))
        assert nxt == runs[0][2]


def test_graph_replayed_in_two_calls(gpu_ctx, hyq):
    """A captured step replayed across generate calls continues the sequence."""
    c = SMALL
    context, prefilled = 64, 10
    model = make_dense_model(c, linear=Q2_0C, seed=4)
    k, v = make_kv_cache(c, context, prefilled, seed=4)
    seqs = []
    for split in (None, 5):
        dec = load_dense(hyq, gpu_ctx, model, context)
        for l in range(c["layers"]):
            dec.load_kv(l, k[l, :prefilled], v[l, :prefilled])
        dec.position = prefilled
        if split is None:
            seqs.append(dec.generate(2, 10))
        else:
            a = dec.generate(2, split)
            b = dec.generate(int(a[-1]), 10 - split)
            seqs.append(np.concatenate([a, b]))
        dec.close()
    assert np.array_equal(seqs[0], seqs[1])


def test_dense_errors(gpu_ctx, hyq):
    c = SMALL
    model = make_dense_model(c, linear=Q2_0C, seed=2)
    dec = load_dense(hyq, gpu_ctx, model, 8)
    dec.position = 8
    with pytest.raises(ValueError):
        dec.forward(1)  # context limit exceeded
    dec.position = 0
    with pytest.raises(ValueError):
        dec.forward(c["vocab"])  # input token outside vocabulary
    with pytest.raises(ValueError):
        dec.generate(1, 9)
    bad = hyq.DenseConfig(2, 500, 4, 1, 128, 1024, 3000, 1e4, 1e-5)
    with pytest.raises(ValueError):
        hyq.DenseDecoder(gpu_ctx, bad, 8)


def test_non_finite_logits_poison_the_session(gpu_ctx, hyq):
    """forward_into rejects non-finite logits and the failed forward poisons
    the session (src/model.rs:348-351, :371, :540-545): an output row whose
    block scale is +inf makes the logits non-finite; the forward fails, so do
    later ones, until a new position starts a new session. The decode loop
    never embeds an out-of-range token meanwhile (the argmax clamps)."""
    c = SMALL
    model = _untied(make_dense_model(c, linear=Q2_0C, seed=12), seed=120)
    out = model["output"].reshape(c["vocab"], -1).copy()
    out[77, 208:210] = np.array([np.inf], np.float16).view(np.uint8)  # Q6_K d of row 77
    model["output"] = out.reshape(-1)
    dec = load_dense(hyq, gpu_ctx, model, 32)
    for call in (lambda: dec.forward(3), lambda: dec.generate(3, 4),
                 lambda: dec.prefill([1, 2, 3])):
        dec.position = 2
        with pytest.raises(ValueError, match="non-finite"):
            call()
        with pytest.raises(ValueError, match="invalidated"):
            dec.forward(3)
    dec.close()


def test_step_argmax_ties_take_the_first_row(gpu_ctx, hyq):
    """The step's greedy token reduces the logits in two passes (per-block
    maxima, then the blocks). Rows 0..776 of the output matrix have zero
    block scales (logits exactly 0) and every later row is a copy of row
    777, so the maximum is tied across many blocks: the token is 777 when
    that logit is positive, else 0 (the first maximum), in forward, the graph
    decode loop and prefill alike."""
    c = SMALL
    model = make_dense_model(c, linear=Q2_0C, seed=13)
    rows = random_matrix(Q6_K, c["vocab"], c["hidden"], seed=130).reshape(c["vocab"], -1)
    rows[777:] = rows[777]
    blocks = rows[:777].reshape(777, -1, 210)  # 210-byte Q6_K blocks, d at 208
    blocks[:, :, 208:210] = np.array([0.0], np.float16).view(np.uint8)
    model["output"] = rows.reshape(-1)
    dec = load_dense(hyq, gpu_ctx, model, 32)
    for token in (3, 5, 8):
        dec.position = 0
        logits, nxt = dec.forward(token)
        assert np.all(logits[:777] == 0) and np.all(logits[777:] == logits[777])
        assert nxt == (777 if logits[777] > 0 else 0), (token, logits[777], nxt)
    dec.position = 0
    toks = dec.generate(3, 6, use_graph=True)
    assert set(int(t) for t in toks) <= {0, 777}
    dec.position = 0
    logits, nxt = dec.prefill([1, 2, 3])
    assert nxt == (777 if logits[777] > 0 else 0)
    dec.close()


@pytest.mark.parametrize("pos,norm_first", [(0, False), (1087, False), (1151, False),
                                            (1087, True), (40, True)])
def test_attention_rope_fused(gpu_ctx, hyq, oracle, pos, norm_first):
    """hyq_attention_rope_d (the decode step's attention launches): RoPE and
    the per-head q/k norms in the dense or the hy_v3 order, the K/V append
    and attention over rows 0..=pos, against the oracle's functions; then
    again at a smaller position with other rows in the same buffers, and
    once with the split partials only (no merge: the output row is left as
    it was), against hyq_attention_d over the appended cache."""
    heads, kvh, D, ctxlen = 16, 4, 128, 1152
    base, eps = 11158840.0, 1e-5
    rng = np.random.default_rng(pos + 7)
    qn = rng.normal(1, 0.02, D).astype(np.float32)
    kn = rng.normal(1, 0.02, D).astype(np.float32)
    kc = rng.normal(0, 1, (ctxlen, kvh * D)).astype(np.float32)
    vc = rng.normal(0, 1, (ctxlen, kvh * D)).astype(np.float32)
    freq = np.array([np.float32(base) ** np.float32(-2.0 * j / D) for j in range(64)],
                    np.float32)
    d = {n: gpu_ctx.array(a) for n, a in dict(qn=qn, kn=kn, freq=freq, kc=kc, vc=vc).items()}
    L = hyq.lib()
    O = oracle.lib()
    scratch = gpu_ctx.empty(L.hyq_attention_scratch_floats(ctxlen, heads), np.float32)
    out = gpu_ctx.empty(heads * D, np.float32)
    kc_ref, vc_ref = kc.copy(), vc.copy()
    for p in (pos, max(pos - 700, 0) // 2):
        q = rng.normal(0, 1, heads * D).astype(np.float32)
        k = rng.normal(0, 1, kvh * D).astype(np.float32)
        v = rng.normal(0, 1, kvh * D).astype(np.float32)
        qd, kd, vd = gpu_ctx.array(q), gpu_ctx.array(k), gpu_ctx.array(v)
        posd = gpu_ctx.array(np.array([p], np.int32))
        hyq.check(L.hyq_attention_rope_d(gpu_ctx.handle, qd.ptr, kd.ptr, vd.ptr, d["qn"].ptr,
                                         d["kn"].ptr, d["freq"].ptr, posd.ptr, ctxlen, heads,
                                         kvh, D, _f(eps), int(norm_first), d["kc"].ptr,
                                         d["vc"].ptr, scratch.ptr, out.ptr))
        c = np.empty(64, np.float32)
        s = np.empty(64, np.float32)
        O.hyqo_rope_tables(128, _f(base), p, c.ctypes.data, s.ctypes.data)

        def rot(x, n, w):
            x = x.copy()
            if norm_first:
                O.hyqo_rms_norm_rows(x.ctypes.data, w.ctypes.data, x.size, 128, _f(eps), 1)
            O.hyqo_rope(x.ctypes.data, n, 128, c.ctypes.data, s.ctypes.data)
            if not norm_first:
                O.hyqo_rms_norm_rows(x.ctypes.data, w.ctypes.data, x.size, 128, _f(eps), 1)
            return x
        q_ref, k_ref = rot(q, heads, qn), rot(k, kvh, kn)
        kc_ref[p], vc_ref[p] = k_ref, v
        ref = np.empty(heads * D, np.float32)
        O.hyqo_attention(q_ref.ctypes.data, kc_ref.ctypes.data, vc_ref.ctypes.data, heads, kvh,
                         D, p + 1, ref.ctypes.data)
        kg, vg = d["kc"].numpy(), d["vc"].numpy()
        assert np.allclose(kg[p], k_ref, rtol=2e-5, atol=2e-6)
        assert np.array_equal(vg[p], v)
        assert np.allclose(kg, kc_ref, rtol=2e-5, atol=2e-6)
        assert np.array_equal(vg, vc_ref)
        got = out.numpy()
        assert np.allclose(got, ref, rtol=2e-5, atol=2e-6), (p, np.abs(got - ref).max())
        assert np.array_equal(qd.numpy(), q)  # the raw query is not modified
    # partials only (out untouched), then hyq_attention_d over the same cache
    hyq.check(L.hyq_attention_rope_d(gpu_ctx.handle, qd.ptr, kd.ptr, vd.ptr, d["qn"].ptr,
                                     d["kn"].ptr, d["freq"].ptr, posd.ptr, ctxlen, heads, kvh,
                                     D, _f(eps), int(norm_first), d["kc"].ptr, d["vc"].ptr,
                                     scratch.ptr, None))
    assert np.array_equal(out.numpy(), got)
    out2 = gpu_ctx.empty(heads * D, np.float32)
    hyq.check(L.hyq_attention_d(gpu_ctx.handle, gpu_ctx.array(q_ref).ptr, d["kc"].ptr,
                                d["vc"].ptr, posd.ptr, ctxlen, heads, kvh, D, scratch.ptr,
                                out2.ptr, None))
    assert np.allclose(out2.numpy(), got, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("kvh,pos", [(4, 0), (4, 31), (4, 32), (4, 1032), (4, 1151), (8, 700),
                                     (1, 500)])
def test_attention_rope_positions_and_repeats(gpu_ctx, hyq, oracle, kvh, pos):
    """hyq_attention_rope_d with its merge at positions that end a split
    (31), start one (32), fill one row (0) and the bench's positions, on 1,
    4 and 8 KV heads: repeated 40 times on the same inputs (the append
    rewrites the same row), every output is bit-identical to the first, and
    it agrees with the oracle's attention (1 to 36 splits)."""
    heads, D, ctxlen = 4 * kvh, 128, 1152
    base, eps = 11158840.0, 1e-5
    rng = np.random.default_rng(pos + kvh)
    qn = rng.normal(1, 0.02, D).astype(np.float32)
    kn = rng.normal(1, 0.02, D).astype(np.float32)
    kc = rng.normal(0, 1, (ctxlen, kvh * D)).astype(np.float32)
    vc = rng.normal(0, 1, (ctxlen, kvh * D)).astype(np.float32)
    q = rng.normal(0, 1, heads * D).astype(np.float32)
    k = rng.normal(0, 1, kvh * D).astype(np.float32)
    v = rng.normal(0, 1, kvh * D).astype(np.float32)
    freq = np.array([np.float32(base) ** np.float32(-2.0 * j / D) for j in range(64)],
                    np.float32)
    d = {n: gpu_ctx.array(a) for n, a in dict(q=q, k=k, v=v, qn=qn, kn=kn, freq=freq, kc=kc,
                                               vc=vc, pos=np.array([pos], np.int32)).items()}
    L = hyq.lib()
    scratch = gpu_ctx.empty(L.hyq_attention_scratch_floats(ctxlen, heads), np.float32)
    out = gpu_ctx.empty(heads * D, np.float32)
    first = None
    for i in range(40):
        hyq.check(L.hyq_attention_rope_d(gpu_ctx.handle, d["q"].ptr, d["k"].ptr, d["v"].ptr,
                                         d["qn"].ptr, d["kn"].ptr, d["freq"].ptr, d["pos"].ptr,
                                         ctxlen, heads, kvh, D, _f(eps), 0, d["kc"].ptr,
                                         d["vc"].ptr, scratch.ptr, out.ptr))
        got = out.numpy()
        if first is None:
            first = got
        assert np.array_equal(got.view(np.uint32), first.view(np.uint32)), (i, pos)
    O = oracle.lib()
    c = np.empty(64, np.float32)
    sn = np.empty(64, np.float32)
    O.hyqo_rope_tables(128, _f(base), pos, c.ctypes.data, sn.ctypes.data)

    def rot(x, n, w):
        x = x.copy()
        O.hyqo_rope(x.ctypes.data, n, 128, c.ctypes.data, sn.ctypes.data)
        O.hyqo_rms_norm_rows(x.ctypes.data, w.ctypes.data, x.size, 128, _f(eps), 1)
        return x
    kc_ref = kc.copy()
    kc_ref[pos] = rot(k, kvh, kn)
    vc_ref = vc.copy()
    vc_ref[pos] = v
    ref = np.empty(heads * D, np.float32)
    q_ref = rot(q, heads, qn)  # (kept alive across the call that reads it)
    O.hyqo_attention(q_ref.ctypes.data, kc_ref.ctypes.data, vc_ref.ctypes.data, heads, kvh, D,
                     pos + 1, ref.ctypes.data)
    assert np.allclose(first, ref, rtol=2e-5, atol=2e-6), np.abs(first - ref).max()


def test_attention_rope_position_at_context_appends_nothing(gpu_ctx, hyq):
    """A device position equal to `context` (which the library cannot check
    on the host) must not be appended past the caches' `context` rows. The
    caches here hold one spare row beyond `context`, so even a wrong append
    stays inside the allocation; the spare row must come back unchanged."""
    heads, kvh, D, ctxlen = 16, 4, 128, 96
    rng = np.random.default_rng(5)
    kc = rng.normal(0, 1, (ctxlen + 1, kvh * D)).astype(np.float32)
    vc = rng.normal(0, 1, (ctxlen + 1, kvh * D)).astype(np.float32)
    arrs = dict(q=rng.normal(0, 1, heads * D), k=rng.normal(0, 1, kvh * D),
                v=rng.normal(0, 1, kvh * D), qn=np.ones(D), kn=np.ones(D),
                freq=np.ones(D // 2), kc=kc, vc=vc)
    d = {n: gpu_ctx.array(np.asarray(a, np.float32)) for n, a in arrs.items()}
    posd = gpu_ctx.array(np.array([ctxlen], np.int32))
    L = hyq.lib()
    scratch = gpu_ctx.empty(L.hyq_attention_scratch_floats(ctxlen, heads), np.float32)
    out = gpu_ctx.empty(heads * D, np.float32)
    hyq.check(L.hyq_attention_rope_d(gpu_ctx.handle, d["q"].ptr, d["k"].ptr, d["v"].ptr,
                                     d["qn"].ptr, d["kn"].ptr, d["freq"].ptr, posd.ptr, ctxlen,
                                     heads, kvh, D, _f(1e-5), 0, d["kc"].ptr, d["vc"].ptr,
                                     scratch.ptr, out.ptr))
    assert np.array_equal(d["kc"].numpy(), kc)
    assert np.array_equal(d["vc"].numpy(), vc)
    assert np.isfinite(out.numpy()).all()
