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
