"""CPU tests: pin the oracle's dense-graph glue (oracle/hyq_oracle_step.c)
before it checks the GPU decoder. The reference's own model tests
(src/model.rs:1096-1125) are restated on the oracle's functions, and the
chunked prefill (forward_into at batch n, src/model.rs:549-616) is pinned to
what fixes it mathematically: in exact arithmetic a chunk of n tokens is n
batch-1 steps, so with f32 activations the two arms may differ only by the
rounding of their different summation orders."""
import ctypes
import math

import numpy as np
import pytest

from synth import Q2_0C, Q6_K, STQ1_0, make_dense_model, make_kv_cache, random_matrix

SMALL = dict(layers=2, hidden=512, heads=4, kv_heads=1, head_dim=128, ffn=1024, vocab=3000,
             rope_base=11158840.0, rms_eps=1e-5)


def _f(x):
    return ctypes.c_float(x)


def _p(a):
    return a.ctypes.data


def test_rotary_pairs_halves_not_neighbors(oracle):
    """src/model.rs:1096-1102: dim 4, frequencies (pi/2, 1), position 1."""
    freqs = np.array([math.pi / 2, 1.0], np.float32)
    ang = freqs * np.float32(1.0)
    cos_s, sin_s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    x = np.array([1.0, 0.0, 0.0, 0.0], np.float32)
    oracle.lib().hyqo_rope(x.ctypes.data, 1, 4, cos_s.ctypes.data, sin_s.ctypes.data)
    assert abs(x[0]) < 1e-6 and x[1] == 0.0 and abs(x[2] - 1.0) < 1e-6


def test_rope_tables_at_position_zero_are_identity(oracle):
    c = np.empty(64, np.float32)
    s = np.empty(64, np.float32)
    oracle.lib().hyqo_rope_tables(128, _f(11158840.0), 0, c.ctypes.data, s.ctypes.data)
    assert np.all(c == 1.0) and np.all(s == 0.0)


def test_causal_attention_does_not_see_future_values(oracle):
    """src/model.rs:1104-1125: two query tokens, two heads sharing one KV
    head of dim 2, zero keys; token t sees positions 0..=t."""
    keys = np.zeros(4, np.float32)
    values = np.array([2.0, 4.0, 100.0, 200.0], np.float32)
    q = np.zeros(4, np.float32)
    got = []
    for t in range(2):
        out = np.empty(4, np.float32)
        oracle.lib().hyqo_attention(q.ctypes.data, keys.ctypes.data, values.ctypes.data, 2, 1,
                                    2, t + 1, out.ctypes.data)
        got.append(out)
    assert np.array_equal(got[0], [2.0, 4.0, 2.0, 4.0])
    assert np.array_equal(got[1], [51.0, 102.0, 51.0, 102.0])


def _rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("n,chunk", [(2, 256), (5, 256), (12, 256), (10, 4), (9, 8)])
def test_prefill_equals_sequential_steps(oracle, n, chunk):
    """Chunks of 2..7 take the reference's row-decode batch arm and >= 8 its
    GEMM arm (src/quant.rs:272-336); a chunk of one token is the batch-1 step
    (the (9, 8) case ends with one)."""
    c = SMALL
    context, past = 40, 7
    model = make_dense_model(c, linear=Q2_0C, seed=3)
    model["output"] = random_matrix(Q6_K, c["vocab"], c["hidden"], 33)
    ref = oracle.DenseOracle(model)
    tokens = np.random.default_rng(n).integers(0, c["vocab"], n).astype(np.int32)
    k1, v1 = make_kv_cache(c, context, past, seed=3)
    k2, v2 = k1.copy(), v1.copy()
    logits = ref.prefill(k1, v1, past, tokens, int8_path=False, chunk=chunk)
    for i, t in enumerate(tokens):
        seq = ref.step(k2, v2, past + i, int(t), int8_path=False)
    assert _rel(logits, seq) <= 2e-5
    span = slice(past, past + n)
    assert _rel(k1[:, span], k2[:, span]) <= 2e-5
    assert _rel(v1[:, span], v2[:, span]) <= 2e-5
    assert np.array_equal(k1[:, :past], k2[:, :past]) and not k1[:, past + n:].any()


def test_prefill_of_one_token_is_the_decode_step(oracle):
    c = SMALL
    model = make_dense_model(c, linear=STQ1_0, seed=4)
    ref = oracle.DenseOracle(model)
    k1, v1 = make_kv_cache(c, 16, 5, seed=4)
    k2, v2 = k1.copy(), v1.copy()
    for int8 in (False, True):
        a = ref.prefill(k1, v1, 5, [17], int8_path=int8)
        b = ref.step(k2, v2, 5, 17, int8_path=int8)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_prefill_errors(oracle):
    c = SMALL
    ref = oracle.DenseOracle(make_dense_model(c, linear=Q2_0C, seed=1))
    k, v = make_kv_cache(c, 8, 0)
    with pytest.raises(ValueError):
        ref.prefill(k, v, 0, [], int8_path=False)
    with pytest.raises(ValueError):
        ref.prefill(k, v, 4, [1, 2, 3, 4, 5], int8_path=False)  # exceeds the context
    with pytest.raises(ValueError):
        ref.prefill(k, v, 0, [1, c["vocab"]], int8_path=False)


# ---- pins of the step glue by what the mathematics fixes ----

@pytest.mark.parametrize("arm", [0, 1], ids=["x86", "aarch64"])
def test_rms_norm_constant_row_closed_form(oracle, arm):
    """rms_norm_into (src/model.rs:785-830): a constant row c has mean square
    c^2, so every output is c * w_i / sqrt(c^2 + eps) up to the rounding of
    the products (each arm rounds twice); a wrong divisor (n - 1, or the sum
    instead of the mean) or a missing eps changes it. The width has a tail
    past the last 16-value step."""
    L = oracle.lib()
    n = 2048 + 5
    w = np.random.default_rng(1).normal(1, 0.02, n).astype(np.float32)
    for c, eps in ((0.75, 1e-5), (3.0, 1e-5), (1e-3, 1e-5), (0.5, 0.0)):
        x = np.full(n, c, np.float32)
        out = np.empty(n, np.float32)
        L.hyqo_rms_norm_into(_p(x), _p(w), n, _f(eps), _p(out), arm)
        exp = c * w.astype(np.float64) / np.sqrt(np.float64(np.float32(c)) ** 2 + eps)
        assert np.allclose(out, exp, rtol=2.5e-7, atol=0), (c, eps)
        # the rows form equals the single-row form row by row
        rows = np.tile(x, 3)
        L.hyqo_rms_norm_rows(_p(rows), _p(w), rows.size, n, _f(eps), arm)
        assert np.array_equal(rows.reshape(3, n), np.tile(out, (3, 1)))


def test_rms_norm_arms_differ_only_in_rounding(oracle):
    """The aarch64 arm forms x * (w * scale) over whole 16-value steps and
    the x86 arm (x * scale) * w (src/model.rs:809, :828): with every w_i a
    power of two both products are exact scalings of one rounded product,
    so the arms agree bit for bit; with general w they differ by at most one
    rounding each (2 ulps); past the last 16-value step the aarch64 arm also
    takes x * scale * w, so the tail agrees bit for bit."""
    L = oracle.lib()
    rng = np.random.default_rng(3)
    n = 2048 + 11
    x = rng.normal(0, 1, n).astype(np.float32)
    out0, out1 = np.empty(n, np.float32), np.empty(n, np.float32)
    w2 = (2.0 ** rng.integers(-3, 4, n)).astype(np.float32)
    L.hyqo_rms_norm_into(_p(x), _p(w2), n, _f(1e-5), _p(out0), 0)
    L.hyqo_rms_norm_into(_p(x), _p(w2), n, _f(1e-5), _p(out1), 1)
    assert np.array_equal(out0.view(np.uint32), out1.view(np.uint32))
    w = rng.normal(1, 0.02, n).astype(np.float32)
    L.hyqo_rms_norm_into(_p(x), _p(w), n, _f(1e-5), _p(out0), 0)
    L.hyqo_rms_norm_into(_p(x), _p(w), n, _f(1e-5), _p(out1), 1)
    body = n // 16 * 16
    assert np.array_equal(out0[body:].view(np.uint32), out1[body:].view(np.uint32))
    ulp = np.spacing(np.abs(out0[:body]))
    assert np.all(np.abs(out0[:body] - out1[:body]) <= 2 * ulp)
    assert not np.array_equal(out0[:body], out1[:body])  # the orders do differ


@pytest.mark.parametrize("arm", [0, 1], ids=["x86", "aarch64"])
def test_rms_norm_power_of_two_invariance(oracle, arm):
    """With eps = 0, scaling the row by 2^k scales the mean square by 4^k and
    its root by 2^k, all exactly, so the output is unchanged bit for bit."""
    L = oracle.lib()
    rng = np.random.default_rng(2)
    n = 6144
    x = rng.normal(0, 1, n).astype(np.float32)
    w = rng.normal(1, 0.02, n).astype(np.float32)
    base = np.empty(n, np.float32)
    L.hyqo_rms_norm_into(_p(x), _p(w), n, _f(0.0), _p(base), arm)
    for k in (-20, -3, 5, 30):
        xs = (x * np.float32(2.0 ** k)).astype(np.float32)
        out = np.empty(n, np.float32)
        L.hyqo_rms_norm_into(_p(xs), _p(w), n, _f(0.0), _p(out), arm)
        assert np.array_equal(out.view(np.uint32), base.view(np.uint32)), k
    # and against float64 within f32 rounding
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5) * w
    out = np.empty(n, np.float32)
    L.hyqo_rms_norm_into(_p(x), _p(w), n, _f(1e-5), _p(out), arm)
    assert np.allclose(out, ref, rtol=1e-5, atol=1e-6)


def test_attention_grouped_query_closed_form(oracle):
    """attention_into (src/model.rs:949-1035) with 8 query heads on 2 KV heads
    of dim 128 and keys along one axis: query head h is sqrt(128) * a_h * e0,
    key p of KV head g is b_{g,p} * e0, so with the 1/sqrt(128) scale the
    score is exactly a_h * b_{g,p} and the softmax weights are known in
    closed form. Each KV head has its own keys and values, so a wrong scale
    or a wrong head map (h % kv_heads instead of h / repeats) fails."""
    L = oracle.lib()
    heads, kvh, D, visible = 8, 2, 128, 5
    rng = np.random.default_rng(3)
    a = np.array([1.0, 0.5, -1.0, 2.0, 0.25, 1.5, -0.5, 1.0])
    b = rng.normal(0, 1, (kvh, visible))
    vals = rng.normal(0, 1, (kvh, visible, D))
    q = np.zeros((heads, D), np.float32)
    q[:, 0] = np.sqrt(128.0) * a
    keys = np.zeros((visible, kvh, D), np.float32)
    keys[:, :, 0] = b.T
    values = np.ascontiguousarray(vals.transpose(1, 0, 2), dtype=np.float32)
    out = np.empty(heads * D, np.float32)
    L.hyqo_attention(_p(q), _p(keys), _p(values), heads, kvh, D, visible, _p(out))
    out = out.reshape(heads, D)
    for h in range(heads):
        g = h // (heads // kvh)
        s = a[h] * b[g].astype(np.float32).astype(np.float64)
        p = np.exp(s - s.max())
        p /= p.sum()
        exp = p @ values[:, g].astype(np.float64)
        assert np.allclose(out[h], exp, rtol=1e-5, atol=1e-6), h


def _rotate(oracle, x, heads, pos, base=11158840.0):
    c = np.empty(64, np.float32)
    s = np.empty(64, np.float32)
    oracle.lib().hyqo_rope_tables(128, _f(base), pos, _p(c), _p(s))
    y = np.ascontiguousarray(x, np.float32).copy()
    oracle.lib().hyqo_rope(_p(y), heads, 128, _p(c), _p(s))
    return y


def test_rope_preserves_pair_norms_and_is_relative(oracle):
    """rope_with_cache (src/model.rs:874-917) rotates each pair (j, j + 64) by
    pos * base^(-2j/128): every pair keeps its length at any position, and the
    product of a rotated query and key depends only on the position
    difference; position 0 is the identity."""
    rng = np.random.default_rng(4)
    q = rng.normal(0, 1, 128).astype(np.float32)
    k = rng.normal(0, 1, 128).astype(np.float32)
    pair = lambda v: v[:64].astype(np.float64) ** 2 + v[64:].astype(np.float64) ** 2
    for pos in (1, 7, 1023, 1151, 40000):
        r = _rotate(oracle, q, 1, pos)
        assert np.allclose(pair(r), pair(q), rtol=1e-5, atol=1e-6), pos
        assert not np.array_equal(r, q)
    dots = []
    for p in (3, 10, 500, 1100):
        for d in (0, 5, 37):
            rq = _rotate(oracle, q, 1, p + d).astype(np.float64)
            rk = _rotate(oracle, k, 1, p).astype(np.float64)
            dots.append((d, float(rq @ rk)))
    for d in (0, 5, 37):
        vals = [v for dd, v in dots if dd == d]
        assert max(vals) - min(vals) <= 2e-3 * max(1.0, abs(vals[0])), (d, vals)
    # positions of one row apply per head: two heads rotate alike
    two = _rotate(oracle, np.concatenate([q, k]), 2, 9)
    assert np.array_equal(two[:128], _rotate(oracle, q, 1, 9))
    assert np.array_equal(two[128:], _rotate(oracle, k, 1, 9))


def _sigmoid(x):
    x = np.float32(x)
    if x >= 0:
        return np.float32(1.0) / (np.float32(1.0) + np.exp(-x))
    e = np.exp(x)
    return e / (np.float32(1.0) + e)


def test_route_closed_forms(oracle):
    """route (src/model.rs:728-767): without normalisation every weight is
    sigmoid(logit) * scale (the bias only selects); with it the weights sum to
    scale unless the selected sigmoids sum below f16's smallest normal
    (6.1035e-5), which then divides instead; equal scores keep index order."""
    logits = np.array([0.0, 2.0, -2.0, 1.0, -30.0, 3.0], np.float32)
    bias = np.array([0.0, 0.0, 10.0, 0.0, 0.0, -5.0], np.float32)
    r = oracle.route(logits, bias, 3, False, 2.5)
    assert [e for e, _ in r] == [2, 1, 3]
    for e, w in r:  # (numpy's and glibc's f32 exp may differ by an ulp)
        assert np.isclose(np.float32(w), _sigmoid(logits[e]) * np.float32(2.5), rtol=3e-7,
                          atol=0), e
    assert oracle.route(np.zeros(4, np.float32), np.zeros(4, np.float32), 2, False,
                        1.0) == [(0, 0.5), (1, 0.5)]  # sigmoid(0) = 1/2 exactly; ties by index
    r = oracle.route(logits, bias, 2, True, 2.826)
    assert abs(sum(w for _, w in r) - 2.826) < 1e-6
    # a softmax route would weight expert 2 by exp(-2)/(exp(-2)+exp(2)), not this
    s2, s1 = _sigmoid(-2.0), _sigmoid(2.0)
    assert abs(r[0][1] - s2 / (s2 + s1) * 2.826) < 1e-6
    # tiny sigmoids: the denominator is floored at f16::MIN_POSITIVE
    tiny = np.array([-20.0, -21.0, -22.0], np.float32)
    r = oracle.route(tiny, np.zeros(3, np.float32), 2, True, 1.0)
    floor = np.float32(6.1035156e-05)
    for e, w in r:
        assert np.isclose(np.float32(w), _sigmoid(tiny[e]) / floor, rtol=3e-7, atol=0), e
    assert abs(sum(w for _, w in r) - 1.0) > 0.5  # not renormalised to the scale


def test_argmax_ties_and_nan(oracle):
    """Greedy sampling (src/generation.rs:281-290): the first maximum wins;
    comparisons with NaN are false, so a NaN is never taken and a NaN at
    index 0 keeps token 0."""
    L = oracle.lib()
    cases = [([1.0, 3.0, 3.0, 2.0], 1), ([np.nan, 5.0, 6.0], 0), ([1.0, np.nan, 0.5], 0),
             ([0.0, np.nan, 2.0, np.nan, 2.0], 2), ([-np.inf] * 4, 0), ([-np.inf, -5.0], 1),
             ([2.0, np.inf, np.inf], 1), ([7.0], 0)]
    for vals, exp in cases:
        x = np.array(vals, np.float32)
        assert L.hyqo_argmax(_p(x), x.size) == exp, vals


@pytest.mark.parametrize("int8", [False, True])
def test_layer_pieces_compose_to_the_step(oracle, int8):
    """The per-layer oracle functions the GPU's traced layers are checked
    against compose to the whole step and the whole chunk bit for bit."""
    c = SMALL
    model = make_dense_model(c, linear=Q2_0C, seed=6)
    model["output"] = random_matrix(Q6_K, c["vocab"], c["hidden"], 66)
    ref = oracle.DenseOracle(model)
    k1, v1 = make_kv_cache(c, 24, 9, seed=6)
    k2, v2 = k1.copy(), v1.copy()
    logits = ref.step(k1, v1, 9, 21, int8_path=int8)
    rb = model["embed"].size // c["vocab"]
    h = oracle.decode(model["embed_dtype"], model["embed"][21 * rb:22 * rb])
    for l in range(c["layers"]):
        h = ref.layer(l, h, k2[l], v2[l], 9, int8_path=int8)
    assert np.array_equal(ref.output(h, int8_path=int8).view(np.uint32), logits.view(np.uint32))
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)
    # batch n
    toks = np.array([5, 17, 2999, 0, 44], np.int32)
    k1, v1 = make_kv_cache(c, 24, 9, seed=6)
    k2, v2 = k1.copy(), v1.copy()
    logits = ref.prefill(k1, v1, 9, toks, int8_path=int8)
    h = np.stack([oracle.decode(model["embed_dtype"], model["embed"][t * rb:(t + 1) * rb])
                  for t in toks])
    for l in range(c["layers"]):
        h = ref.prefill_layer(l, h, k2[l], v2[l], 9).reshape(toks.size, -1)
    assert np.array_equal(ref.output(h[-1], int8_path=int8).view(np.uint32),
                          logits.view(np.uint32))
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)


# ---- the MoE FFN and the hy_v3 order ----

HYV3_SMALL = dict(layers=2, hidden=512, heads=4, kv_heads=1, head_dim=128, ffn=1024, vocab=3000,
                  rope_base=11158840.0, rms_eps=1e-5)
MOE_SMALL = dict(experts=8, used=2, mid=256, shared_mid=512, normalize=True, scale=2.5)


def _hyv3(seed=0, **kw):
    from synth import Q4_K, Q8_0, make_hyv3_model
    moe = dict(MOE_SMALL, **kw)
    return make_hyv3_model(HYV3_SMALL, moe, linear=Q4_K, expert=Q4_K, shared=Q8_0, seed=seed)


def _ffn64(oracle, dg, dd, g, u, d, hidden, mid, x):
    """f64 DenseFfn::forward of rows x over golden-pinned decoded weights."""
    G = oracle.decode(dg, g).reshape(mid, hidden).astype(np.float64)
    U = oracle.decode(dg, u).reshape(mid, hidden).astype(np.float64)
    D = oracle.decode(dd, d).reshape(hidden, mid).astype(np.float64)
    a, b = x @ G.T, x @ U.T
    return ((a / (1.0 + np.exp(-a))) * b) @ D.T


def _moe64(oracle, e, hidden, x):
    """Moe::forward (src/model.rs:687-726) in f64 from pinned pieces: the F32
    router product, route (pinned above), the shared expert and each chosen
    expert's FFN, added in ascending expert order."""
    x64 = x.astype(np.float64)
    logits = (x64 @ e["router"].astype(np.float64).T).astype(np.float32)
    out = _ffn64(oracle, e["dtype_shared"], e["dtype_shared_down"], e["sgate"], e["sup"],
                 e["sdown"], hidden, e["shared_mid"], x64)
    E, mid = e["experts"], e["mid"]
    gb, db = e["gate"].size // E, e["down"].size // E
    for t in range(x.shape[0]):
        for ex, w in sorted(oracle.route(logits[t], e["bias"], e["used"], e["normalize"],
                                         e["scale"])):
            out[t] += w * _ffn64(oracle, e["dtype_gate"], e["dtype_down"],
                                 e["gate"][ex * gb:(ex + 1) * gb], e["up"][ex * gb:(ex + 1) * gb],
                                 e["down"][ex * db:(ex + 1) * db], hidden, mid, x64[t:t + 1])[0]
    return out


@pytest.mark.parametrize("n", [1, 6])
def test_moe_forward_matches_f64_chain(oracle, n):
    model = _hyv3(seed=3)
    e = model["layers"][1]["moe"]
    H = HYV3_SMALL["hidden"]
    x = np.random.default_rng(n).normal(0, 1, (n, H)).astype(np.float32)
    ref = _moe64(oracle, e, H, x)
    got = oracle.moe_forward(e, H, x, n, int8_path=False)
    assert _rel(got, ref) <= 2e-6, _rel(got, ref)
    if n == 1:
        # the int8 arm: every product from Q8 activations (~1/127 of a value)
        q = oracle.moe_forward(e, H, x, 1, int8_path=True)
        assert 1e-5 < _rel(q, ref) <= 3e-2, _rel(q, ref)


def test_moe_forward_single_expert_identity(oracle):
    """One expert, used 1, normalised: the weight is sigmoid/sigmoid * scale =
    scale exactly, so with scale 1 the output is shared(x) + expert(x) - the
    same f32 operations as two dense FFNs (in both arms)."""
    model = _hyv3(seed=4, experts=1, used=1, scale=1.0)
    e = model["layers"][1]["moe"]
    H = HYV3_SMALL["hidden"]
    x = np.random.default_rng(9).normal(0, 1, (1, H)).astype(np.float32)
    from synth import Q4_K, Q8_0
    for int8 in (False, True):
        got = oracle.moe_forward(e, H, x, 1, int8_path=int8)
        sh = oracle.moe_forward(dict(e, scale=1e-30), H, x, 1, int8_path=int8)  # ~shared only
        ex = got - sh
        ref = _ffn64(oracle, Q4_K, Q4_K, e["gate"], e["up"], e["down"], H, e["mid"],
                     x.astype(np.float64))
        assert _rel(ex, ref) <= (3e-2 if int8 else 1e-5), int8
        shref = _ffn64(oracle, Q8_0, Q8_0, e["sgate"], e["sup"], e["sdown"], H,
                       e["shared_mid"], x.astype(np.float64))
        assert _rel(sh, shref) <= (3e-2 if int8 else 1e-5), int8


@pytest.mark.parametrize("arch", [0, 1])
def test_qk_norm_order_by_architecture(oracle, arch):
    """hy_v3 normalises q and k per head before RoPE, hunyuan-dense after it
    (src/model.rs:425-446): the K row the layer appends equals an f64
    restatement of the chosen order, and not of the other one."""
    model = _hyv3(seed=5)
    model["arch"] = arch
    c = HYV3_SMALL
    ref = oracle.DenseOracle(model)
    H, D, pos = c["hidden"], 128, 7
    kc = np.zeros((16, D), np.float32)
    vc = np.zeros((16, D), np.float32)
    h = np.random.default_rng(1).normal(0, 1, H).astype(np.float32)
    ref.layer(0, h, kc, vc, pos, int8_path=False)
    L = model["layers"][0]
    xn = h.astype(np.float64) / np.sqrt(np.mean(h.astype(np.float64) ** 2) + 1e-5)
    xn = xn * L["attn_norm"]
    k = oracle.decode(model["linear"], L["k"]).reshape(D, H).astype(np.float64) @ xn
    freq = np.float32(c["rope_base"]) ** (-2.0 * np.arange(64, dtype=np.float64) / 128)
    ang = pos * freq.astype(np.float32).astype(np.float64)
    cs, sn = np.cos(ang), np.sin(ang)

    def rope(v):
        return np.concatenate([v[:64] * cs - v[64:] * sn, v[:64] * sn + v[64:] * cs])

    def norm(v):
        return v / np.sqrt(np.mean(v ** 2) + 1e-5) * L["k_norm"]

    exp = rope(norm(k)) if arch == 1 else norm(rope(k))
    other = norm(rope(k)) if arch == 1 else rope(norm(k))
    assert _rel(kc[pos], exp) <= 1e-5
    assert _rel(kc[pos], other) > 1e-3


# ---- the Q8 tap the decode-path parity tests replace codes through ----

@pytest.mark.parametrize("moe", [False, True])
def test_q8_tap_records_and_replays_the_int8_path(oracle, moe):
    """hyqo_layer_step_tap / hyqo_output_logits_tap / hyqo_moe_forward_tap:
    each recorded stage's codes and scales are the quantizer's output on the
    recorded input; replaying the recorded codes gives the untapped layer,
    output and MoE FFN bit for bit; and one replaced code reaches the
    product: it moves the layer's output, its K/V row or a later stage's
    recorded input (with every stage replaced, a later stage's codes absorb
    an earlier stage's change, which its recorded input still shows)."""
    c = HYV3_SMALL if moe else SMALL
    model = _hyv3(seed=7) if moe else make_dense_model(c, linear=Q2_0C, seed=7)
    ref = oracle.DenseOracle(model)
    k, v = make_kv_cache(c, 24, 9, seed=7)
    h = np.random.default_rng(7).normal(0, 1, c["hidden"]).astype(np.float32)
    for l in range(c["layers"]):
        widths = ref.stages(l)
        kk, vv = k[l].copy(), v[l].copy()
        plain = ref.layer(l, h, kk, vv, 9, int8_path=True)
        out, tap = ref.layer_tap(l, h, k[l].copy(), v[l].copy(), 9)
        assert np.array_equal(out.view(np.uint32), plain.view(np.uint32))
        use = {}
        for st, n in enumerate(widths):
            x, q, s = tap.own(st, n)
            q_ref, s_ref = oracle.q8_quantize(x)
            assert np.array_equal(q, q_ref) and np.array_equal(s, s_ref), (l, st)
            use[st] = (q.copy(), s.copy())
        again, _ = ref.layer_tap(l, h, k[l].copy(), v[l].copy(), 9, use=use)
        assert np.array_equal(again.view(np.uint32), plain.view(np.uint32))
        for st in range(len(widths)):
            moved = {a: (b[0].copy(), b[1]) for a, b in use.items()}
            q = moved[st][0]
            j = int(np.argmax(np.abs(q) < 120))
            q[j] += 1
            kk2, vv2 = k[l].copy(), v[l].copy()
            changed, tap2 = ref.layer_tap(l, h, kk2, vv2, 9, use=moved)
            later = [not np.array_equal(tap2.own(a, widths[a])[0], tap.own(a, widths[a])[0])
                     for a in range(st + 1, len(widths))]
            assert (not np.array_equal(changed, plain) or any(later) or
                    not np.array_equal(kk2, kk) or not np.array_equal(vv2, vv)), (l, st)
        with pytest.raises(ValueError):
            ref.layer_tap(l, h, k[l].copy(), v[l].copy(), 9,
                          use={a: b for a, b in use.items() if a != 1})
        h = plain
    logits = ref.output(h, int8_path=True)
    lg, tap = ref.output_tap(h)
    assert np.array_equal(lg.view(np.uint32), logits.view(np.uint32))
    x, q, s = tap.own(0, c["hidden"])
    lg2, _ = ref.output_tap(h, use={0: (q.copy(), s.copy())})
    assert np.array_equal(lg2.view(np.uint32), logits.view(np.uint32))
    if moe:
        e = model["layers"][1]["moe"]
        xr = np.random.default_rng(8).normal(0, 1, (1, c["hidden"])).astype(np.float32)
        plain = oracle.moe_forward(e, c["hidden"], xr, 1, int8_path=True)[0]
        out, tap = oracle.moe_forward_tap(e, c["hidden"], xr)
        assert np.array_equal(out.view(np.uint32), plain.view(np.uint32))
        st = [oracle.STAGE_FFN_IN, oracle.STAGE_DOWN_IN] + \
            [oracle.STAGE_EXPERT_DOWN_IN + j for j in range(e["used"])]
        n = [c["hidden"], e["shared_mid"]] + [e["mid"]] * e["used"]
        use = {a: tuple(t.copy() for t in tap.own(a, w)[1:]) for a, w in zip(st, n)}
        again, _ = oracle.moe_forward_tap(e, c["hidden"], xr, use=use)
        assert np.array_equal(again.view(np.uint32), plain.view(np.uint32))
