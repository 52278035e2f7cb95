"""GPU parity of the chunked prefill (hyq_dense_prefill: Model::prefill_into
and the batch > 1 arm of forward_into, src/model.rs:549-646) and of its
batched causal attention against the oracle, through the C ABI.

Tolerances (floating point, stated per test): the batched attention within
rtol 1e-5, atol 1e-6 of the oracle, as the one-token attention (its matrix
products carry f16 operand pairs hi + lo, within 2^-21 of f32). The
prefill's products round activations and weights to f16 (2^-11 relative
each) where the oracle's batched products are f32, so the
last row's logits and the appended K/V rows are held to 1e-2 relative in the
2-norm. A one-token prompt takes the batch-1 step: bit-identical to
hyq_dense_forward."""
import numpy as np
import pytest

import q8_proof as P

from synth import (Q2_0C, Q4_K, Q6_K, Q8_0, STQ1_0, load_dense, make_dense_model, make_kv_cache,
                   random_matrix)

pytestmark = pytest.mark.gpu

SMALL = dict(layers=2, hidden=512, heads=4, kv_heads=1, head_dim=128, ffn=1024, vocab=3000,
             rope_base=11158840.0, rms_eps=1e-5)


def _print(*a):
    print(*a, flush=True)


def _rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def _attention_rows(hyq, gpu_ctx, q, kc, vc, pos, n, heads, kvh):
    L = hyq.lib()
    ctxlen = kc.shape[0]
    qd, kd, vd = gpu_ctx.array(q), gpu_ctx.array(kc), gpu_ctx.array(vc)
    posd = gpu_ctx.array(np.array([pos], np.int32))
    scratch = gpu_ctx.empty(L.hyq_attention_rows_scratch_floats(ctxlen, heads, n), np.float32)
    out = gpu_ctx.empty(n * heads * 128, np.float32)
    hyq.check(L.hyq_attention_rows_d(gpu_ctx.handle, qd.ptr, kd.ptr, vd.ptr, posd.ptr, n,
                                     ctxlen, heads, kvh, 128, scratch.ptr, out.ptr))
    return out.numpy().reshape(n, heads * 128)


@pytest.mark.parametrize("pos,n,heads,kvh", [(0, 1, 16, 4), (0, 37, 16, 4), (100, 64, 16, 4),
                                             (1000, 152, 16, 4), (5, 256, 16, 4),
                                             (70, 200, 4, 4), (33, 99, 8, 4), (300, 45, 12, 4),
                                             (0, 300, 16, 4)])
def test_attention_rows_matches_oracle(gpu_ctx, hyq, oracle, pos, n, heads, kvh):
    """Query heads per KV head 4, 1, 2 and 3; chunks from 1 to 300 rows."""
    D, ctxlen = 128, 1152
    _print("attention_rows", pos, n, heads, kvh)
    rng = np.random.default_rng(pos * 1000 + n)
    q = rng.normal(0, 1, (n, heads * D)).astype(np.float32)
    kc = rng.normal(0, 1, (ctxlen, kvh * D)).astype(np.float32)
    vc = rng.normal(0, 1, (ctxlen, kvh * D)).astype(np.float32)
    got = _attention_rows(hyq, gpu_ctx, q, kc, vc, pos, n, heads, kvh)
    for i in range(n):
        ref = np.empty(heads * D, np.float32)
        oracle.lib().hyqo_attention(q[i].ctypes.data, kc.ctypes.data, vc.ctypes.data, heads,
                                    kvh, D, pos + i + 1, ref.ctypes.data)
        assert np.allclose(got[i], ref, rtol=1e-5, atol=1e-6), (i, np.abs(got[i] - ref).max())


def test_attention_rows_do_not_see_future_values(gpu_ctx, hyq):
    """src/model.rs:1104-1125 at head_dim 128: zero queries and keys, two
    rows at positions 0 and 1 average the values they can see."""
    heads, kvh, D = 2, 1, 128
    vc = np.zeros((2, D), np.float32)
    vc[0, :2] = [2.0, 4.0]
    vc[1, :2] = [100.0, 200.0]
    got = _attention_rows(hyq, gpu_ctx, np.zeros((2, heads * D), np.float32),
                          np.zeros((2, D), np.float32), vc, 0, 2, heads, kvh)
    o = got.reshape(2, heads, D)
    assert np.array_equal(o[0, :, :2], [[2.0, 4.0], [2.0, 4.0]])
    assert np.array_equal(o[1, :, :2], [[51.0, 102.0], [51.0, 102.0]])
    assert not o[:, :, 2:].any()


def _model(linear, seed):
    c = SMALL
    model = make_dense_model(c, linear=linear, seed=seed)
    model["output"] = random_matrix(Q6_K, c["vocab"], c["hidden"], seed + 50)
    return model


def _decoder(hyq, gpu_ctx, model, context, past, seed):
    c = model["cfg"]
    dec = load_dense(hyq, gpu_ctx, model, context)
    k, v = make_kv_cache(c, context, past, seed=seed)
    for l in range(c["layers"]):
        dec.load_kv(l, k[l, :past], v[l, :past])
    dec.position = past
    return dec, k, v


@pytest.mark.parametrize("linear,n", [(Q2_0C, 2), (Q2_0C, 37), (Q2_0C, 300), (STQ1_0, 9),
                                      (STQ1_0, 256), (Q2_0C, 257)])
def test_prefill_matches_oracle(gpu_ctx, hyq, oracle, linear, n):
    """The oracle runs 300 tokens as chunks of 256 and 44 (PREFILL_CHUNK,
    src/model.rs:18), 257 as 256 and a batch-1 step."""
    c = SMALL
    context, past = 320, 5
    _print("prefill", linear, n)
    model = _model(linear, seed=7)
    dec, k, v = _decoder(hyq, gpu_ctx, model, context, past, seed=7)
    tokens = np.random.default_rng(n).integers(0, c["vocab"], n).astype(np.int32)
    logits, nxt = dec.prefill(tokens)
    assert dec.position == past + n
    ref = oracle.DenseOracle(model)
    ref_logits = ref.prefill(k, v, past, tokens, int8_path=True)
    rel = _rel(logits, ref_logits)
    _print("  logits rel", rel)
    assert rel <= 1e-2, rel
    assert nxt == int(np.argmax(logits))
    top = np.sort(ref_logits)[-2:]
    if top[1] - top[0] > 2e-2 * np.abs(ref_logits).max():
        assert nxt == int(np.argmax(ref_logits))
    for l in range(c["layers"]):
        kg, vg = dec.read_kv(l, past + n)
        assert np.array_equal(kg[:past], k[l, :past]) and np.array_equal(vg[:past], v[l, :past])
        rk, rv = _rel(kg[past:], k[l, past:past + n]), _rel(vg[past:], v[l, past:past + n])
        _print("  layer", l, "kv rel", rk, rv)
        assert rk <= 1e-2 and rv <= 1e-2, (l, rk, rv)
    dec.close()


def test_prefill_results_do_not_depend_on_the_pass_size(gpu_ctx, hyq):
    c = SMALL
    model = _model(Q2_0C, seed=6)
    tokens = np.random.default_rng(6).integers(0, c["vocab"], 300).astype(np.int32)
    runs = []
    for rows in (1024, 64, 7, 1):
        dec, _, _ = _decoder(hyq, gpu_ctx, model, 320, 4, seed=6)
        dec.set_prefill_rows(rows)
        logits, nxt = dec.prefill(tokens)
        kv = [dec.read_kv(l, 304) for l in range(c["layers"])]
        runs.append((logits, nxt, kv))
        dec.close()
    for logits, nxt, kv in runs[1:]:
        assert nxt == runs[0][1]
        assert np.array_equal(logits.view(np.uint32), runs[0][0].view(np.uint32))
        for (k, v), (k0, v0) in zip(kv, runs[0][2]):
            assert np.array_equal(k.view(np.uint32), k0.view(np.uint32))
            assert np.array_equal(v.view(np.uint32), v0.view(np.uint32))


def test_prompt_of_256k_plus_1_ends_with_the_decode_step(gpu_ctx, hyq):
    """src/model.rs:642-644: the last of 257 tokens is a one-token chunk."""
    c = SMALL
    model = _model(Q2_0C, seed=5)
    tokens = np.random.default_rng(5).integers(0, c["vocab"], 257).astype(np.int32)
    a, _, _ = _decoder(hyq, gpu_ctx, model, 300, 2, seed=5)
    b, _, _ = _decoder(hyq, gpu_ctx, model, 300, 2, seed=5)
    la, ta = a.prefill(tokens)
    b.prefill(tokens[:256], want_logits=False)
    lb, tb = b.forward(int(tokens[256]))
    assert ta == tb and np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    a.close()
    b.close()


def test_prefill_of_one_token_is_the_decode_step(gpu_ctx, hyq):
    c = SMALL
    model = _model(Q2_0C, seed=8)
    a, _, _ = _decoder(hyq, gpu_ctx, model, 32, 11, seed=8)
    b, _, _ = _decoder(hyq, gpu_ctx, model, 32, 11, seed=8)
    la, ta = a.prefill([123])
    lb, tb = b.forward(123)
    assert ta == tb and np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    assert a.position == b.position == 12
    for l in range(c["layers"]):
        for x, y in zip(a.read_kv(l, 12), b.read_kv(l, 12)):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    a.close()
    b.close()


def test_decode_continues_after_prefill(gpu_ctx, hyq, oracle):
    """Batch-1 steps after a prefill attend to the prefilled rows: each
    step's logits match the oracle's int8 step on the GPU's own cache and
    int8 codes (the decode bar, 1e-4 relative; tests/q8_proof.py)."""
    c = SMALL
    context, past, n = 64, 3, 40
    model = _model(Q2_0C, seed=9)
    dec, _, _ = _decoder(hyq, gpu_ctx, model, context, past, seed=9)
    tokens = np.random.default_rng(1).integers(0, c["vocab"], n).astype(np.int32)
    _, token = dec.prefill(tokens)
    ref = oracle.DenseOracle(model)
    kvw = c["kv_heads"] * c["head_dim"]
    gpu_ctx.set_q8_trace(1 << 20)
    for i in range(3):
        pos = past + n + i
        k = np.zeros((c["layers"], context, kvw), np.float32)
        v = np.zeros_like(k)
        for l in range(c["layers"]):
            k[l, :pos], v[l, :pos] = dec.read_kv(l, pos)
        gpu_ctx.clear_q8_trace()
        logits, nxt = dec.forward(token)
        P.check_step(gpu_ctx, ref, model, c, k, v, pos, token, logits, nxt, f"step {i}")
        token = nxt
    gpu_ctx.set_q8_trace(None)
    assert dec.position == past + n + 3
    dec.close()


def test_prefill_errors(gpu_ctx, hyq):
    c = SMALL
    model = _model(Q2_0C, seed=2)
    dec, _, _ = _decoder(hyq, gpu_ctx, model, 16, 4, seed=2)
    with pytest.raises(ValueError):
        dec.prefill([])  # prompt must contain at least one token
    with pytest.raises(ValueError):
        dec.prefill(np.arange(13))  # prompt exceeds context limit
    with pytest.raises(ValueError):
        dec.prefill([1, c["vocab"]])  # input token outside vocabulary
    assert dec.position == 4
    _, t = dec.prefill(np.arange(12))  # exactly fills the context
    assert dec.position == 16
    dec.close()


MIXED = dict(SMALL, ffn=6144)  # 24 groups: the down projection runs as three K slices


@pytest.mark.parametrize("linear,down", [(Q4_K, Q6_K), (Q8_0, Q8_0), (Q6_K, Q6_K)])
def test_mixed_formats_prefill_and_decode(gpu_ctx, hyq, oracle, linear, down):
    """The Q4_K_M mix (Q4_K linears, Q6_K down) and single-format Q8_0 / Q6_K
    models: prefill within 1e-2 and the following decode steps within 1e-4
    (on the GPU's own cache and int8 codes) of the oracle."""
    c = MIXED
    _print("mixed", linear, down)
    model = make_dense_model(c, linear=linear, down=down, seed=31)
    model["output"] = random_matrix(Q6_K, c["vocab"], c["hidden"], 81)
    context, past, n = 48, 6, 30
    dec, k, v = _decoder(hyq, gpu_ctx, model, context, past, seed=31)
    tokens = np.random.default_rng(31).integers(0, c["vocab"], n).astype(np.int32)
    logits, token = dec.prefill(tokens)
    ref = oracle.DenseOracle(model)
    rel = _rel(logits, ref.prefill(k, v, past, tokens, int8_path=True))
    _print("  prefill rel", rel)
    assert rel <= 1e-2, rel
    kvw = c["kv_heads"] * c["head_dim"]
    gpu_ctx.set_q8_trace(1 << 20)
    for i in range(2):
        pos = past + n + i
        kc = np.zeros((c["layers"], context, kvw), np.float32)
        vc = np.zeros_like(kc)
        for l in range(c["layers"]):
            kc[l, :pos], vc[l, :pos] = dec.read_kv(l, pos)
        gpu_ctx.clear_q8_trace()
        step_logits, nxt = dec.forward(token)
        P.check_step(gpu_ctx, ref, model, c, kc, vc, pos, token, step_logits, nxt,
                     f"mixed step {i}")
        token = nxt
    gpu_ctx.set_q8_trace(None)
    dec.close()
