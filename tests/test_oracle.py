"""CPU tests: pin the oracle against the reference's golden vectors, closed
forms and invariants before the GPU path is compared with it."""
import json
import math
import os

import numpy as np
import pytest

from synth import (BLOCK_BYTES, BLOCK_LEN, Q2_0C, Q4_K, Q6_K, Q8_0, QUANT, STQ1_0, NAMES,
                   random_blocks, random_matrix, row_bytes, set_block_scale)

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def load_quant_json():
    with open(os.path.join(GOLDEN, "quant.json")) as f:
        return json.load(f)


# ---- decoders: tests/quant_reference.rs:12-50 over tests/fixtures/quant.json ----

@pytest.mark.parametrize("case", load_quant_json(), ids=lambda c: c["dtype"])
def test_decoders_match_golden_bits(oracle, case):
    dt = oracle.NAMES[case["dtype"]]
    encoded = bytes.fromhex(case["encoded_hex"])
    expected = np.array(case["expected_f32_bits"], dtype=np.uint32)
    got = oracle.decode(dt, encoded)
    assert got.size == expected.size
    bad = np.nonzero(got.view(np.uint32) != expected)[0]
    assert bad.size == 0, f"{case['dtype']} lanes {bad[:8]}"
    # the fixture's dot check: |dot - f64 oracle| < 1e-3 + 1e-4*|oracle|
    x = np.sin(np.arange(got.size, dtype=np.float32) * np.float32(0.17)).astype(np.float32)
    ref = float(np.dot(expected.view(np.float32).astype(np.float64), x.astype(np.float64)))
    assert abs(oracle.dot(got, x) - ref) < 1e-3 + 1e-4 * abs(ref)


def test_decode_rejects_partial_blocks(oracle):
    with pytest.raises(ValueError):
        oracle.decode(Q2_0C, bytes(130), 256)  # partial output block
    with pytest.raises(ValueError):
        oracle.decode(STQ1_0, bytes(41), 256)  # wrong byte count


# ---- closed forms: src/quant.rs:2602-2644 ----

def test_q2_codes_and_scale(oracle):
    block = bytearray([0b11100100] * 130)
    block[0:2] = np.array([0.5], dtype=np.float16).tobytes()
    out = oracle.decode(Q2_0C, bytes(block))
    assert np.array_equal(out.reshape(-1, 4), np.tile([-1.5, -0.5, 0.5, 1.5], (128, 1)))


def test_stq_all_patterns_and_stride(oracle):
    block = bytearray(42)
    block[40:42] = np.array([2.0], dtype=np.float16).tobytes()
    for g in range(64):
        block[g // 2] |= (g % 16) << (4 * (g % 2))
        block[32 + g // 8] |= (g // 16 % 2) << (g % 8)
    out = oracle.decode(STQ1_0, bytes(block))
    for g in range(64):
        zero, tail, nz = (g % 16) // 4, g % 4, 0
        for p in range(4):
            if p == zero:
                expected = 0.0
            else:
                sign = 1.0 if nz == 0 or tail & (1 << (nz - 1)) == 0 else -1.0
                nz += 1
                expected = sign * (2.0 if g // 16 % 2 == 0 else -2.0)
            assert out[g // 16 * 64 + g % 16 + 16 * p] == expected


def test_stq_codebook_has_exactly_one_zero_per_group(oracle):
    # every codebook entry has exactly one zero digit -> exactly 25% zeros
    blocks = random_blocks(STQ1_0, 64, seed=3)
    set_block_scale(STQ1_0, blocks, 1.0)
    d = oracle.decode(STQ1_0, blocks).reshape(64, 4, 4, 16)  # block, c, p, g%16
    zeros = (d == 0).sum(axis=2)
    assert np.all(zeros == 1)


# ---- dot: src/quant.rs:2646-2654 ----

@pytest.mark.parametrize("n", [0, 1, 3, 7, 16, 32, 127, 256, 512, 2049])
def test_vector_dot_matches_scalar_with_tails(oracle, n):
    a = np.sin(np.arange(n, dtype=np.float32) * np.float32(0.7)).astype(np.float32)
    b = np.cos(np.arange(n, dtype=np.float32) * np.float32(0.9)).astype(np.float32)
    assert abs(oracle.dot(a, b) - oracle.dot_scalar(a, b)) < 1e-4


# ---- fused f32 row dots vs decode+dot: src/quant.rs:2656-2711 ----

@pytest.mark.parametrize("dtype", [STQ1_0, Q6_K, Q2_0C])
def test_fused_row_dot_matches_decode(oracle, dtype):
    bl, bb = BLOCK_LEN[dtype], BLOCK_BYTES[dtype]
    for seed in range(64):
        block = bytearray(bb)
        mul = 2654435761 if dtype == STQ1_0 else 40503
        step = 7 if dtype == STQ1_0 else 13
        rng_range = range(40) if dtype == STQ1_0 else (range(208) if dtype == Q6_K
                                                        else range(2, 130))
        for i in rng_range:
            block[i] = (seed * mul + i * step) & 0xFF
        scale = (1.0 + seed % 0.5) if dtype == STQ1_0 else (0.25 + seed % 0.75)
        off = {STQ1_0: 40, Q6_K: 208, Q2_0C: 0}[dtype]
        block[off:off + 2] = np.array([scale], dtype=np.float16).tobytes()
        k = {STQ1_0: 0.31, Q6_K: 0.17, Q2_0C: 0.17}[dtype]
        f = np.cos if dtype == STQ1_0 else np.sin
        x = f((np.arange(bl, dtype=np.float32) + np.float32(seed)) * np.float32(k)).astype(
            np.float32)
        dec = oracle.decode(dtype, bytes(block))
        assert abs(oracle.row_dot_f32(dtype, np.frombuffer(bytes(block), np.uint8), bl, x)
                   - oracle.dot(dec, x)) < 1e-3, seed


# ---- Q8 activations: src/quant.rs:2955-2978 plus constructed vectors ----

def q8_case_arrays(c):
    """Inputs and scales of a q8_vectors.json case from their f32 bit patterns."""
    x = np.array([int(b, 16) for b in c["x_bits"]], np.uint32).view(np.float32)
    s = np.array([int(b, 16) for b in c["scales_bits"]], np.uint32).view(np.float32)
    return x, np.array(c["q"], np.int8), s


def test_q8_constructed_vectors(oracle):
    """Ties, saturation, zero groups, tails, and NaN / infinity in the steps
    and in the tail (max_abs_neon's FMAX propagates NaN, f32::max skips it)."""
    with open(os.path.join(GOLDEN, "q8_vectors.json")) as f:
        cases = json.load(f)
    names = {c["name"] for c in cases}
    assert {"nan_in_body", "nan_in_tail", "nan_in_body_with_tail", "infinity"} <= names
    for c in cases:
        x, q_ref, s_ref = q8_case_arrays(c)
        q, s = oracle.q8_quantize(x)
        assert np.array_equal(q, q_ref), c["name"]
        assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32)), c["name"]


def test_q8_round_trip_invariant(oracle):
    values = (np.sin(np.arange(1024, dtype=np.float32) * np.float32(0.37)) * 3).astype(
        np.float32)
    q, s = oracle.q8_quantize(values)
    assert s.size == 4
    for g in range(4):
        restored = q[g * 256:(g + 1) * 256].astype(np.float32) * s[g]
        err = np.abs(restored - values[g * 256:(g + 1) * 256])
        assert np.all(err <= s[g] * 0.5 + 1e-6)
    q, s = oracle.q8_quantize(np.zeros(256, dtype=np.float32))
    assert s.tolist() == [0.0] and not q.any()


def test_q8_deinterleave_q2c_permutation(oracle):
    q = np.arange(-64, 64, dtype=np.int8)
    out = oracle.q8_deinterleave_q2c(q)
    for c in range(2):
        for k in range(4):
            for j in range(16):
                assert out[64 * c + 16 * k + j] == q[64 * c + 4 * j + k]


# ---- integer block sums: pinned to the golden-pinned decoder with unit scales ----

def _int_weights(oracle, dtype, blocks, mode=None):
    """Integer weights from the decoder with scales forced to 1 (exact)."""
    b = blocks.copy()
    if dtype == Q4_K:
        set_block_scale(Q4_K, b, 1.0 if mode == "A" else 0.0, 0.0 if mode == "A" else 1.0)
    elif dtype == Q6_K:
        set_block_scale(Q6_K, b, 1.0)
        b.reshape(-1, 210)[:, 192:208] = 1
    else:
        set_block_scale(dtype, b, 1.0)
    w = oracle.decode(dtype, b)
    assert np.all(w == np.round(w))
    return w.astype(np.int64)


@pytest.mark.parametrize("dtype", QUANT, ids=lambda d: NAMES[d])
def test_isums_equal_integer_sums_over_decoder(oracle, dtype):
    cols = 1024
    blocks = random_matrix(dtype, 1, cols, seed=dtype)
    x = np.random.default_rng(7).normal(0, 1, cols).astype(np.float32)
    q, _ = oracle.q8_quantize(x)
    got = oracle.row_isums(dtype, blocks, cols, q)
    qa = q.astype(np.int64)
    if dtype == Q4_K:
        wa = _int_weights(oracle, dtype, blocks, "A")
        wb = _int_weights(oracle, dtype, blocks, "B")
        exp = []
        for b in range(cols // 256):
            sl = slice(b * 256, (b + 1) * 256)
            exp += [int((wa[sl] * qa[sl]).sum()), -int((wb[sl] * qa[sl]).sum())]
    else:
        w = _int_weights(oracle, dtype, blocks)
        unit = {Q2_0C: 256, STQ1_0: 256, Q8_0: 32}.get(dtype)
        if dtype == Q6_K:
            # plane k of block b covers chunk*128 + p*32 + half*16 + (0..15)
            exp = []
            for b in range(cols // 256):
                planes = [0] * 16
                for chunk in range(2):
                    for p in range(4):
                        for hf in range(2):
                            o = b * 256 + chunk * 128 + p * 32 + hf * 16
                            planes[chunk * 8 + 2 * p + hf] = int(
                                (w[o:o + 16] * qa[o:o + 16]).sum())
                exp += planes
        else:
            exp = [int((w[i:i + unit] * qa[i:i + unit]).sum()) for i in range(0, cols, unit)]
    assert got.tolist() == exp


@pytest.mark.parametrize("dtype", QUANT, ids=lambda d: NAMES[d])
def test_int8_gemv_oracle_matches_bruteforce(oracle, dtype):
    rows, cols = 16, 2048
    w = random_matrix(dtype, rows, cols, seed=11 + dtype)
    x = np.random.default_rng(5).normal(0, 1, cols).astype(np.float32)
    q, s = oracle.q8_quantize(x)
    y, mag = oracle.gemv_q8_f64(dtype, w, rows, cols, q, s)
    yb, magb = oracle.gemv_q8_bruteforce(dtype, w, rows, cols, q, s)
    assert np.allclose(mag, magb, rtol=1e-12)
    assert np.all(np.abs(y - yb) <= 1e-6 * mag)


def test_int8_reference_recipe(oracle):
    """The inputs of sdot_kernels_match_int8_reference (src/quant.rs:2983-3078)."""
    for seed in range(8):
        x = (np.sin((np.arange(512, dtype=np.float32) + np.float32(seed)) * np.float32(0.11))
             * 2).astype(np.float32)
        x[:256] *= 1.0
        x[256:] *= 2.0
        q, s = oracle.q8_quantize(x)
        stq = np.array([(seed * 2654435761 + i * 7) & 0xFF for i in range(84)], np.uint8)
        stq[40:42] = np.array([0.5], np.float16).view(np.uint8)
        stq[82:84] = np.array([0.25], np.float16).view(np.uint8)
        q6 = np.array([(seed * 40503 + i * 13) & 0xFF for i in range(420)], np.uint8)
        q6[208:210] = np.array([0.125], np.float16).view(np.uint8)
        q6[418:420] = np.array([0.75], np.float16).view(np.uint8)
        q2c = np.array([(seed * 40503 + i * 13) & 0xFF for i in range(130)], np.uint8)
        q2c[0:2] = np.array([0.375], np.float16).view(np.uint8)
        for dt, blob in ((STQ1_0, stq), (Q6_K, q6), (Q2_0C, q2c)):
            y, mag = oracle.gemv_q8_f64(dt, blob, 1, 512, q, s)
            yb, _ = oracle.gemv_q8_bruteforce(dt, blob, 1, 512, q, s)
            assert abs(y[0] - yb[0]) <= mag[0] * 1e-5


# ---- Weight::matmul x86 paths vs the f64 brute force ----

@pytest.mark.parametrize("dtype", QUANT, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("batch", [1, 3, 9])
def test_matmul_paths_match_f64(oracle, dtype, batch):
    rows, cols = 72, 1024
    w = random_matrix(dtype, rows, cols, seed=dtype + batch)
    x = np.random.default_rng(batch).normal(0, 1, batch * cols).astype(np.float32)
    y = oracle.matmul(dtype, w, rows, cols, x, batch, threads=2)
    yr, mag = oracle.matmul_f64(dtype, w, rows, cols, x, batch)
    assert np.all(np.abs(y - yr) <= 1e-5 * mag)


@pytest.mark.parametrize("dtype", QUANT, ids=lambda d: NAMES[d])
def test_gate_up_silu_matches_two_products(oracle, dtype):
    rows, cols = 40, 512
    g = random_matrix(dtype, rows, cols, seed=1)
    u = random_matrix(dtype, rows, cols, seed=2)
    x = np.random.default_rng(3).normal(0, 1, cols).astype(np.float32)
    y = oracle.gate_up_silu(dtype, g, u, rows, cols, x, threads=2)
    gr, _ = oracle.matmul_f64(dtype, g, rows, cols, x, 1)
    ur, _ = oracle.matmul_f64(dtype, u, rows, cols, x, 1)
    with np.errstate(over="ignore"):
        ref = gr[0] / (1 + np.exp(-gr[0])) * ur[0]
    assert np.allclose(y, ref, rtol=1e-4, atol=1e-6)


def test_chunk_rows(oracle):
    L = oracle.lib()
    assert L.hyqo_chunk_rows(6144, 8) == 384
    assert L.hyqo_chunk_rows(100, 8) == 32
    assert L.hyqo_chunk_rows(1 << 20, 8) == 2048
    assert L.hyqo_chunk_rows(3 * 33, 1) == 50  # odd -> rounded up to even


# ---- MoE routing: src/model.rs:1088-1094 ----

def test_routing_bias_changes_selection_not_weights(oracle):
    r = oracle.route(np.array([0.0, 2.0, -2.0]), np.array([0.0, 0.0, 10.0]), 2, True, 2.826)
    assert [e for e, _ in r] == [2, 1]
    assert abs(sum(w for _, w in r) - 2.826) < 1e-6
    assert r[0][1] < r[1][1]


def test_routing_ties_break_by_index(oracle):
    r = oracle.route(np.zeros(6), np.zeros(6), 3, False, 1.0)
    assert [e for e, _ in r] == [0, 1, 2]
    assert all(w == 0.5 for _, w in r)


def test_moe_experts_match_dense_products(oracle):
    hidden, mid, experts, tokens = 256, 256, 3, 5
    gate = random_matrix(Q4_K, experts * mid, hidden, seed=1)
    up = random_matrix(Q4_K, experts * mid, hidden, seed=2)
    down = random_matrix(Q4_K, experts * hidden, mid, seed=3)
    x = np.random.default_rng(0).normal(0, 1, tokens * hidden).astype(np.float32)
    pt = np.array([0, 1, 2, 3, 4, 0, 2], np.int32)
    pe = np.array([0, 0, 0, 1, 1, 2, 2], np.int32)
    pw = np.array([0.5, 0.25, 1.0, 0.75, 0.1, 0.3, 0.2], np.float32)
    out = oracle.moe_experts(Q4_K, Q4_K, gate, up, down, experts, hidden, mid, x, pt, pe, pw,
                             np.zeros(tokens * hidden, np.float32), threads=2)
    ref = np.zeros((tokens, hidden))
    gb, db = row_bytes(Q4_K, hidden) * mid, row_bytes(Q4_K, mid) * hidden
    for t, e, wgt in zip(pt, pe, pw):
        xt = x[t * hidden:(t + 1) * hidden]
        g, _ = oracle.matmul_f64(Q4_K, gate[e * gb:(e + 1) * gb], mid, hidden, xt, 1)
        u, _ = oracle.matmul_f64(Q4_K, up[e * gb:(e + 1) * gb], mid, hidden, xt, 1)
        with np.errstate(over="ignore"):
            h = (g[0] / (1 + np.exp(-g[0])) * u[0]).astype(np.float32)
        d, _ = oracle.matmul_f64(Q4_K, down[e * db:(e + 1) * db], hidden, mid, h, 1)
        ref[t] += wgt * d[0]
    assert np.allclose(out.reshape(tokens, hidden), ref, rtol=1e-3, atol=1e-5)


def test_f16_conversion_edge_cases(oracle):
    L = oracle.lib()
    for bits in (0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xC000, 0x7BFF, 0x7C00, 0xFC00):
        ref = float(np.array([bits], np.uint16).view(np.float16)[0])
        got = L.hyqo_f16_to_f32(bits)
        assert (got == ref) and (math.copysign(1, got) == math.copysign(1, ref))
    assert math.isnan(L.hyqo_f16_to_f32(0x7E00))
