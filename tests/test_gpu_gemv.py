"""GPU parity of the int8 decode path: HIP kernels through the C ABI against
the oracle on the same seeded inputs.

Bars: decoders and Q8 bit-exact; integer block sums bit-exact; f32 outputs
within the reference's own bound |err| <= 1e-5 * sum|w q s| per row and
1e-4 relative in the 2-norm (tests/gpu_util.py:check_decode_path)."""
import json
import os

import numpy as np
import pytest

from gpu_util import check_decode_path, device_bytes
from synth import (NAMES, Q2_0C, Q4_K, Q6_K, Q8_0, QUANT, STQ1_0, random_matrix, row_bytes)

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _print(*a):
    print(*a, flush=True)


# ---- decoders ----

def test_decode_golden_bits_on_gpu(gpu_ctx, oracle):
    with open(os.path.join(GOLDEN, "quant.json")) as f:
        cases = json.load(f)
    for c in cases:
        _print("decode", c["dtype"])
        dt = oracle.NAMES[c["dtype"]]
        got = gpu_ctx.decode(dt, bytes.fromhex(c["encoded_hex"]))
        exp = np.array(c["expected_f32_bits"], np.uint32)
        assert np.array_equal(got.view(np.uint32), exp), c["dtype"]


@pytest.mark.parametrize("dtype", QUANT, ids=lambda d: NAMES[d])
def test_weight_rows_decode_bit_exact(gpu_ctx, oracle, hyq, dtype):
    rows, cols = 24, 1024
    w = random_matrix(dtype, rows, cols, seed=100 + dtype)
    W = gpu_ctx.upload(dtype, w, (cols, rows))
    rb = row_bytes(dtype, cols)
    for r in (0, 7, rows - 1):
        got = W.row(r)
        ref = oracle.decode(dtype, w[r * rb:(r + 1) * rb])
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (NAMES[dtype], r)


def test_stq_all_patterns_on_gpu(gpu_ctx, oracle):
    block = bytearray(42)
    block[40:42] = np.array([2.0], np.float16).tobytes()
    for g in range(64):
        block[g // 2] |= (g % 16) << (4 * (g % 2))
        block[32 + g // 8] |= (g // 16 % 2) << (g % 8)
    got = gpu_ctx.decode(STQ1_0, bytes(block))
    assert np.array_equal(got, oracle.decode(STQ1_0, bytes(block)))
    W = gpu_ctx.upload(STQ1_0, np.frombuffer(bytes(block), np.uint8), (256, 1))
    assert np.array_equal(W.row(0), got)


# ---- Q8 activations ----

def test_quantize_q8_bit_exact(gpu_ctx, hyq, oracle):
    cases = json.load(open(os.path.join(GOLDEN, "q8_vectors.json")))
    rng = np.random.default_rng(0)
    inputs = [np.array([int(b, 16) for b in c["x_bits"]], np.uint32).view(np.float32)
              for c in cases]
    inputs += [rng.normal(0, 1, 2048).astype(np.float32),
               (rng.normal(0, 3, 6144) * (np.arange(6144) % 7)).astype(np.float32),
               rng.normal(0, 1, 264).astype(np.float32)]
    for x in inputs:
        _print("quantize", x.size)
        n = x.size
        q8 = gpu_ctx.q8(n)
        xd = gpu_ctx.array(x)
        q8.quantize_into(xd.ptr)
        gpu_ctx.sync()
        q_dev = device_bytes(hyq, gpu_ctx, q8.values_ptr, n)
        s_dev = device_bytes(hyq, gpu_ctx, q8.scales_ptr, 4 * ((n + 255) // 256))
        q_ref, s_ref = oracle.q8_quantize(x)
        assert np.array_equal(q_dev.view(np.int8), q_ref)
        assert np.array_equal(s_dev.view(np.uint32), s_ref.view(np.uint32))
    # the golden cases' own answers too (the NaN and infinity rules included)
    for c, x in zip(cases, inputs):
        q8 = gpu_ctx.q8(x.size)
        q8.quantize_into(gpu_ctx.array(x).ptr)
        gpu_ctx.sync()
        q_dev = device_bytes(hyq, gpu_ctx, q8.values_ptr, x.size).view(np.int8)
        s_dev = device_bytes(hyq, gpu_ctx, q8.scales_ptr, 4 * ((x.size + 255) // 256))
        assert np.array_equal(q_dev, np.array(c["q"], np.int8)), c["name"]
        s_ref = np.array([int(b, 16) for b in c["scales_bits"]], np.uint32)
        assert np.array_equal(s_dev.view(np.uint32), s_ref), c["name"]


# ---- integer block sums ----

SHAPES = {Q2_0C: (3072, 2048), STQ1_0: (3072, 2048), Q4_K: (6144, 2048),
          Q6_K: (2048, 2048), Q8_0: (2048, 2048)}


@pytest.mark.parametrize("dtype", QUANT, ids=lambda d: NAMES[d])
def test_isums_bit_exact(gpu_ctx, hyq, oracle, dtype):
    rows, cols = SHAPES[dtype]
    rows = min(rows, 1024)
    _print("isums", NAMES[dtype], rows, cols)
    w = random_matrix(dtype, rows, cols, seed=7 + dtype)
    x = np.random.default_rng(dtype).normal(0, 1, cols).astype(np.float32)
    W = gpu_ctx.upload(dtype, w, (cols, rows))
    q8 = gpu_ctx.q8(cols)
    xd = gpu_ctx.array(x)
    q8.quantize_into(xd.ptr)
    per = hyq.isums_per_row(dtype, cols)
    out = gpu_ctx.empty(rows * per, np.int32)
    hyq.check(hyq.lib().hyq_gemv_isums_d(gpu_ctx.handle, W.handle, q8.handle, out.ptr))
    got = out.numpy().reshape(rows, per)
    q_ref, _ = oracle.q8_quantize(x)
    ref = oracle.isums(dtype, w, rows, cols, q_ref)
    assert np.array_equal(got, ref)


# ---- f32 outputs ----

@pytest.mark.parametrize("dtype", QUANT, ids=lambda d: NAMES[d])
def test_gemv_matches_oracle(gpu_ctx, oracle, dtype):
    rows, cols = SHAPES[dtype]
    _print("gemv", NAMES[dtype], rows, cols)
    w = random_matrix(dtype, rows, cols, seed=21 + dtype)
    x = np.random.default_rng(3 + dtype).normal(0, 1, cols).astype(np.float32)
    W = gpu_ctx.upload(dtype, w, (cols, rows))
    y = W.matmul(x, 1)
    q, s = oracle.q8_quantize(x)
    y_ref, mag = oracle.gemv_q8_f64(dtype, w, rows, cols, q, s)
    check_decode_path(y, y_ref, mag, NAMES[dtype])


@pytest.mark.parametrize("dtype", [Q2_0C, STQ1_0], ids=lambda d: NAMES[d])
@pytest.mark.parametrize("rows,cols", [(2048, 2048), (12288, 2048)],
                         ids=["attn_out_2048x2048", "gate_up_12288x2048"])
def test_gemv_c2_shapes(gpu_ctx, oracle, dtype, rows, cols):
    """The 1.8B attention output and stacked gate+up matrices at their own
    sizes (the QKV and down shapes are above), Q8 input, against the
    oracle's f64 dot on the same codes."""
    _print("c2", NAMES[dtype], rows, cols)
    w = random_matrix(dtype, rows, cols, seed=61)
    x = np.random.default_rng(62).normal(0, 1, cols).astype(np.float32)
    y = gpu_ctx.upload(dtype, w, (cols, rows)).matmul(x, 1)
    q, s = oracle.q8_quantize(x)
    y_ref, mag = oracle.gemv_q8_f64(dtype, w, rows, cols, q, s)
    check_decode_path(y, y_ref, mag, NAMES[dtype])


@pytest.mark.parametrize("dtype", QUANT, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("rows,cols", [(2048, 6144), (3071, 4096), (4100, 4096)],
                         ids=["2048x6144", "3071x4096", "4100x4096"])
def test_gemv_k6144_down_shape(gpu_ctx, oracle, dtype, rows, cols):
    """Under 4096 rows of 16-31 groups the GEMV gives each row 16 lanes (one
    or two groups each; the 1.8B down projection's shape and a ragged one);
    Q6_K does so at any row count (4100 rows), the other formats keep 8."""
    _print("down", NAMES[dtype], rows, cols)
    w = random_matrix(dtype, rows, cols, seed=5)
    x = np.random.default_rng(9).normal(0, 1, cols).astype(np.float32)
    y = gpu_ctx.upload(dtype, w, (cols, rows)).matmul(x, 1)
    q, s = oracle.q8_quantize(x)
    y_ref, mag = oracle.gemv_q8_f64(dtype, w, rows, cols, q, s)
    check_decode_path(y, y_ref, mag, NAMES[dtype])


@pytest.mark.parametrize("dtype", QUANT, ids=lambda d: NAMES[d])
def test_gemv_wide_rows(gpu_ctx, hyq, oracle, dtype):
    """Rows of at least 32 groups with few rows (a 7B down-projection shape,
    shortened) take the kernel with 32 lanes per row: 36 groups (some lanes
    hold two, some one), a ragged last workgroup; both the f32-input launch
    (matmul, which for Q2_0C takes the half-group kernel at this row count)
    and the Q8-input launch."""
    rows, cols = 1001, 36 * 256
    _print("wide", NAMES[dtype])
    w = random_matrix(dtype, rows, cols, seed=31 + dtype)
    x = np.random.default_rng(11 + dtype).normal(0, 1, cols).astype(np.float32)
    W = gpu_ctx.upload(dtype, w, (cols, rows))
    y = W.matmul(x, 1)
    q, s = oracle.q8_quantize(x)
    y_ref, mag = oracle.gemv_q8_f64(dtype, w, rows, cols, q, s)
    check_decode_path(y, y_ref, mag, NAMES[dtype])
    q8 = gpu_ctx.q8(cols)
    xd = gpu_ctx.array(x)
    q8.quantize_into(xd.ptr)
    yd = gpu_ctx.empty(rows, np.float32)
    hyq.check(hyq.lib().hyq_gemv_q8_d(gpu_ctx.handle, W.handle, q8.handle, None, yd.ptr))
    check_decode_path(yd.numpy(), y_ref, mag, NAMES[dtype] + " q8 input")


@pytest.mark.parametrize("rows", [1, 7, 8, 9, 63, 65, 513])
def test_gemv_ragged_rows(gpu_ctx, oracle, rows):
    cols = 512
    w = random_matrix(Q2_0C, rows, cols, seed=rows)
    x = np.random.default_rng(rows).normal(0, 1, cols).astype(np.float32)
    y = gpu_ctx.upload(Q2_0C, w, (cols, rows)).matmul(x, 1)
    q, s = oracle.q8_quantize(x)
    y_ref, mag = oracle.gemv_q8_f64(Q2_0C, w, rows, cols, q, s)
    check_decode_path(y, y_ref, mag, f"rows={rows}")


def test_gemv_zero_activation_group(gpu_ctx, oracle):
    rows, cols = 64, 1024
    w = random_matrix(STQ1_0, rows, cols, seed=1)
    x = np.random.default_rng(2).normal(0, 1, cols).astype(np.float32)
    x[256:512] = 0.0  # an all-zero group: scale 0, values 0
    y = gpu_ctx.upload(STQ1_0, w, (cols, rows)).matmul(x, 1)
    q, s = oracle.q8_quantize(x)
    assert s[1] == 0.0
    y_ref, mag = oracle.gemv_q8_f64(STQ1_0, w, rows, cols, q, s)
    check_decode_path(y, y_ref, mag)


def test_lm_head_q6k_full_size(gpu_ctx, hyq, oracle):
    """The f32 row (quantized in the launch, two rows per lane) and the Q8
    row (one row per lane) give the same bits, within the oracle's bound."""
    rows, cols = 120818, 2048
    _print("lm_head")
    w = random_matrix(Q6_K, rows, cols, seed=77)
    x = np.random.default_rng(77).normal(0, 1, cols).astype(np.float32)
    W = gpu_ctx.upload(Q6_K, w, (cols, rows))
    y = W.matmul(x, 1)
    q, s = oracle.q8_quantize(x)
    y_ref, mag = oracle.gemv_q8_f64(Q6_K, w, rows, cols, q, s)
    check_decode_path(y, y_ref, mag, "lm_head")
    q8 = gpu_ctx.q8(cols)
    xd = gpu_ctx.array(x)
    q8.quantize_into(xd.ptr)
    yd = gpu_ctx.empty(rows, np.float32)
    hyq.check(hyq.lib().hyq_gemv_q8_d(gpu_ctx.handle, W.handle, q8.handle, None, yd.ptr))
    assert np.array_equal(yd.numpy().view(np.uint32), y.view(np.uint32))


# ---- fused entry points ----

@pytest.mark.parametrize("dtype", [Q2_0C, STQ1_0, Q6_K], ids=lambda d: NAMES[d])
def test_fused_qkv_equals_three_products(gpu_ctx, hyq, dtype):
    """src/quant.rs:2806-2822: the fused projections equal separate products."""
    cols = 2048
    ws = [random_matrix(dtype, r, cols, seed=s) for r, s in ((2048, 1), (512, 2), (512, 3))]
    W = [gpu_ctx.upload(dtype, w, (cols, w.size // row_bytes(dtype, cols))) for w in ws]
    x = np.random.default_rng(4).normal(0, 1, cols).astype(np.float32)
    fq, fk, fv = hyq.Weight.gemv_qkv(W[0], W[1], W[2], x)
    for fused, w in zip((fq, fk, fv), W):
        assert np.array_equal(fused, w.matmul(x, 1))


@pytest.mark.parametrize("dtype", QUANT, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("cols", [2048, 4096])
def test_gate_up_silu(gpu_ctx, oracle, dtype, cols):
    """8 groups per row and 16. At 8 groups the fused launch and the plain
    GEMV both give a row 8 lanes, so each half of the product equals the
    plain GEMV (the SiLU within 2e-6); at 16 the plain GEMV gives a row 16
    lanes and the fused one 8 or 16 by format, so the sums may round in
    another order. Either way the product is checked against the oracle's
    f64 halves on the same Q8 input (relative 2-norm 1e-4)."""
    rows = 1536
    g = random_matrix(dtype, rows, cols, seed=31)
    u = random_matrix(dtype, rows, cols, seed=32)
    x = np.random.default_rng(33).normal(0, 1, cols).astype(np.float32)
    G = gpu_ctx.upload(dtype, g, (cols, rows))
    U = gpu_ctx.upload(dtype, u, (cols, rows))
    y = G.matmul_gate_up_silu(U, x)
    gy, uy = G.matmul(x, 1), U.matmul(x, 1)
    if cols == 2048:
        with np.errstate(over="ignore"):
            exp = ((gy / (np.float32(1) + np.exp(-gy))) * uy).astype(np.float32)
        assert np.allclose(y, exp, rtol=2e-6, atol=0), NAMES[dtype]
    q, s = oracle.q8_quantize(x)
    gr, gm = oracle.gemv_q8_f64(dtype, g, rows, cols, q, s)
    ur, um = oracle.gemv_q8_f64(dtype, u, rows, cols, q, s)
    check_decode_path(gy, gr, gm)
    check_decode_path(uy, ur, um)
    with np.errstate(over="ignore"):
        ref = gr / (1 + np.exp(-gr)) * ur
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel <= 1e-4, (NAMES[dtype], cols, rel)


@pytest.mark.parametrize("dtype", QUANT, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("cols", [256, 1536, 2048, 6144, 8704, 16384])
def test_staged_gemv_equals_quantize_then_gemv(gpu_ctx, hyq, dtype, cols):
    """hyq_matmul_d at batch 1 quantizes the f32 row inside the GEMV launch
    (one 32-lane half wave per 256-value group; rows above 32 groups take the
    looped stage). Its output equals hyq_quantize_q8_d + hyq_gemv_q8_d bit for
    bit: the same maxima, IEEE divisions, round-half-even and exact integer
    sums. A row 4 bytes off float4 alignment takes the two-launch path and
    must agree as well. An all-zero group (scale 0) is included, and from
    three groups on a group holding a NaN: the reference's NEON maximum
    (FMAX) makes that group's maximum NaN, so its scale and codes are 0 and
    the product equals that of the same row with the group zeroed."""
    if cols % hyq.lib().hyq_block_len(dtype):
        pytest.skip("width is not a whole number of blocks")
    rows = 200
    _print("staged", NAMES[dtype], cols)
    w = random_matrix(dtype, rows, cols, seed=cols + dtype)
    rng = np.random.default_rng(cols)
    x = (rng.normal(0, 1, cols) * rng.choice([1e-3, 1.0, 40.0], cols)).astype(np.float32)
    x[256:512] = 0.0
    nan_group = cols >= 768
    if nan_group:
        x[600] = np.nan
    W = gpu_ctx.upload(dtype, w, (cols, rows))
    xd = gpu_ctx.array(np.concatenate([x, x[:4]]))
    xo = gpu_ctx.array(np.concatenate([np.zeros(1, np.float32), x]))  # x at byte offset 4
    y_staged, y_two, y_off = (gpu_ctx.empty(rows, np.float32) for _ in range(3))
    L = hyq.lib()
    hyq.check(L.hyq_matmul_d(gpu_ctx.handle, W.handle, xd.ptr, 1, y_staged.ptr))
    hyq.check(L.hyq_matmul_d(gpu_ctx.handle, W.handle, xo.ptr + 4, 1, y_off.ptr))
    q8 = gpu_ctx.q8(cols)
    q8.quantize_into(xd.ptr)
    hyq.check(L.hyq_gemv_q8_d(gpu_ctx.handle, W.handle, q8.handle, None, y_two.ptr))
    a, b, c = y_staged.numpy(), y_two.numpy(), y_off.numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(c.view(np.uint32), b.view(np.uint32))
    if nan_group:
        assert np.isfinite(a).all()
        xz = x.copy()
        xz[512:768] = 0.0
        yz = gpu_ctx.empty(rows, np.float32)
        hyq.check(L.hyq_matmul_d(gpu_ctx.handle, W.handle, gpu_ctx.array(xz).ptr, 1, yz.ptr))
        assert np.array_equal(a.view(np.uint32), yz.numpy().view(np.uint32))


def test_residual_epilogue(gpu_ctx, hyq, oracle):
    rows, cols = 2048, 2048
    w = random_matrix(Q2_0C, rows, cols, seed=8)
    x = np.random.default_rng(8).normal(0, 1, cols).astype(np.float32)
    h = np.random.default_rng(9).normal(0, 1, rows).astype(np.float32)
    W = gpu_ctx.upload(Q2_0C, w, (cols, rows))
    q8 = gpu_ctx.q8(cols)
    xd, hd = gpu_ctx.array(x), gpu_ctx.array(h)
    yd = gpu_ctx.empty(rows, np.float32)
    q8.quantize_into(xd.ptr)
    hyq.check(hyq.lib().hyq_gemv_q8_d(gpu_ctx.handle, W.handle, q8.handle, hd.ptr, yd.ptr))
    y = yd.numpy()
    plain = W.matmul(x, 1)
    assert np.array_equal(y, h + plain)


def test_expert_view_equals_separate_upload(gpu_ctx):
    cols, rows, E = 2048, 512, 4
    w = random_matrix(Q4_K, rows * E, cols, seed=12)
    x = np.random.default_rng(12).normal(0, 1, cols).astype(np.float32)
    W = gpu_ctx.upload(Q4_K, w, (cols, rows, E))
    eb = rows * row_bytes(Q4_K, cols)
    for e in range(E):
        view = W.expert(e)
        alone = gpu_ctx.upload(Q4_K, w[e * eb:(e + 1) * eb], (cols, rows))
        assert view.shape() == (cols, rows)
        assert np.array_equal(view.matmul(x, 1), alone.matmul(x, 1))
    with pytest.raises(ValueError):
        W.expert(E)


def test_failed_allocation_leaves_later_launches_alone(gpu_ctx, hyq):
    """A device allocation past the device's memory fails with HYQ_ENOMEM, and
    the runtime error it leaves is not reported by the next (good) launch:
    every launcher checks the runtime's last error after launching."""
    w = random_matrix(Q2_0C, 64, 512, seed=3)
    W = gpu_ctx.upload(Q2_0C, w, (512, 64))
    x = np.random.default_rng(3).normal(0, 1, 512).astype(np.float32)
    y0 = W.matmul(x, 1)
    for attempt in range(2):
        _print("allocation of 2^50 bytes, attempt", attempt)
        with pytest.raises(hyq.HyqError) as e:
            gpu_ctx.empty(1 << 48, np.float32)
        assert e.value.code == hyq.ENOMEM
        assert np.array_equal(W.matmul(x, 1), y0)
    W.release()


def test_shape_errors(gpu_ctx, hyq):
    w = random_matrix(Q2_0C, 8, 512, seed=0)
    with pytest.raises(ValueError):
        gpu_ctx.upload(Q2_0C, w[:-1], (512, 8))  # wrong byte count
    W = gpu_ctx.upload(Q2_0C, w, (512, 8))
    with pytest.raises(ValueError):
        W.matmul(np.zeros(511, np.float32), 1)
    with pytest.raises(ValueError):
        W.row(8)
    with pytest.raises(ValueError):
        gpu_ctx.decode(Q2_0C, bytes(129), 512)
