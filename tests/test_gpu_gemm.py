"""GPU parity of the batched (prefill) path: Weight::matmul at batch >= 2
(src/quant.rs:272-344) through the C ABI against the oracle's f64 brute force
of decoded weights x f32 activations (oracle/hyq_oracle.c:hyqo_matmul_f64).

Tolerance of the f16-MFMA path (tests/gpu_util.py:check_prefill_path): per
element |err| <= 2e-3 * sum|w x| (f16 rounding of both operands bounds each
term's relative error by 2*2^-11 < 1e-3) and 2e-3 relative in the 2-norm."""
import numpy as np
import pytest

from gpu_util import check_prefill_path
from synth import NAMES, Q2_0C, Q4_K, Q6_K, Q8_0, QUANT, STQ1_0, random_matrix, row_bytes

pytestmark = pytest.mark.gpu


def _print(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("dtype", QUANT, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("batch", [2, 7, 8, 130])
def test_matmul_batched_matches_oracle(gpu_ctx, oracle, dtype, batch):
    rows, cols = 200, 1024  # a ragged last row tile (200 = 128 + 72)
    _print("gemm", NAMES[dtype], rows, cols, batch)
    w = random_matrix(dtype, rows, cols, seed=40 + dtype + batch)
    x = np.random.default_rng(batch).normal(0, 1, batch * cols).astype(np.float32)
    W = gpu_ctx.upload(dtype, w, (cols, rows))
    y = W.matmul(x, batch).reshape(batch, rows)
    y_ref, mag = oracle.matmul_f64(dtype, w, rows, cols, x, batch)
    check_prefill_path(y, y_ref, mag, f"{NAMES[dtype]} batch {batch}")


@pytest.mark.parametrize("dtype", [Q4_K, Q6_K], ids=lambda d: NAMES[d])
def test_prefill_7b_k4096_block(gpu_ctx, oracle, dtype):
    """A 7B-shaped slice: K = 4096, 512 tokens, 384 weight rows."""
    rows, cols, batch = 384, 4096, 512
    _print("gemm 7B slice", NAMES[dtype])
    w = random_matrix(dtype, rows, cols, seed=7)
    x = np.random.default_rng(7).normal(0, 1, batch * cols).astype(np.float32)
    y = gpu_ctx.upload(dtype, w, (cols, rows)).matmul(x, batch).reshape(batch, rows)
    y_ref, mag = oracle.matmul_f64(dtype, w, rows, cols, x, batch)
    check_prefill_path(y, y_ref, mag, NAMES[dtype])


@pytest.mark.parametrize("dtype,rows,cols", [(Q4_K, 14336, 4096), (Q6_K, 4096, 14336),
                                             (Q4_K, 6144, 4096)],
                         ids=["gate_up_q4k", "down_q6k", "qkv_q4k"])
def test_prefill_7b_full_size_sampled_rows(gpu_ctx, oracle, dtype, rows, cols):
    """Full 7B prefill GEMMs at 512 tokens; a seeded sample of 96 weight rows
    (all 512 tokens each) is checked against the oracle, which is row-local."""
    batch = 512
    _print("gemm full", NAMES[dtype], rows, cols)
    w = random_matrix(dtype, rows, cols, seed=rows)
    x = np.random.default_rng(cols).normal(0, 1, batch * cols).astype(np.float32)
    y = gpu_ctx.upload(dtype, w, (cols, rows)).matmul(x, batch).reshape(batch, rows)
    assert np.all(np.isfinite(y))
    rb = row_bytes(dtype, cols)
    pick = np.sort(np.random.default_rng(5).choice(rows, 96, replace=False))
    pick[-1] = rows - 1
    sub = np.concatenate([w[r * rb:(r + 1) * rb] for r in pick])
    y_ref, mag = oracle.matmul_f64(dtype, sub, len(pick), cols, x, batch)
    check_prefill_path(y[:, pick], y_ref, mag, NAMES[dtype])


@pytest.mark.parametrize("dtype,rows,cols,batch", [(Q4_K, 14336, 4096, 300), (Q6_K, 4096, 14336, 270),
                                                   (Q4_K, 6144, 4096, 257), (Q4_K, 6112, 4096, 300)],
                         ids=["gate_up_q4k_300", "down_q6k_270", "qkv_q4k_257", "rows96_partial_300"])
def test_prefill_7b_ragged_token_blocks(gpu_ctx, oracle, dtype, rows, cols, batch):
    """The 256-token tiles with their activations in fragment order at token
    counts that end inside a 32-token block (and inside a 256-token tile):
    sampled weight rows, all tokens, against the oracle; the partial block's
    rows past the batch feed sums that are never written. [6144 x 4096] and
    [6112 x 4096] run as 96-row tiles (the latter's last tile 64 rows)."""
    _print("gemm ragged", NAMES[dtype], rows, cols, batch)
    w = random_matrix(dtype, rows, cols, seed=rows + batch)
    x = np.random.default_rng(batch).normal(0, 1, batch * cols).astype(np.float32)
    y = gpu_ctx.upload(dtype, w, (cols, rows)).matmul(x, batch).reshape(batch, rows)
    assert np.all(np.isfinite(y))
    rb = row_bytes(dtype, cols)
    pick = np.sort(np.random.default_rng(6).choice(rows, 64, replace=False))
    pick[-1] = rows - 1
    sub = np.concatenate([w[r * rb:(r + 1) * rb] for r in pick])
    y_ref, mag = oracle.matmul_f64(dtype, sub, len(pick), cols, x, batch)
    check_prefill_path(y[:, pick], y_ref, mag, NAMES[dtype])


def test_fragment_tiles_equal_row_tiles(gpu_ctx):
    """At 300 tokens a [14336 x 4096] product runs as 256-token tiles with its
    activations in fragment order; at 200 tokens the same weight runs as
    128-token tiles with its activations copied through LDS. The same
    operands meet in the same k order either way, so the first 200 token rows
    agree bit for bit."""
    rows, cols = 14336, 4096
    w = random_matrix(Q4_K, rows, cols, seed=11)
    x = np.random.default_rng(11).normal(0, 1, 300 * cols).astype(np.float32)
    W = gpu_ctx.upload(Q4_K, w, (cols, rows))
    big = W.matmul(x, 300).reshape(300, rows)
    small = W.matmul(x[:200 * cols], 200).reshape(200, rows)
    assert np.array_equal(big[:200].view(np.uint32), small.view(np.uint32))
    W.release()


def test_batched_rows_are_independent_of_batch(gpu_ctx):
    """Each token's output row does not depend on the other tokens of the
    batch, for batches on the same side of one 128-token tile: above it the
    K split is a rule on the weight's shape (here none); at or below it the
    row tiles alone leave CUs idle and K is split in two (a 128-token tile
    boundary and partial tiles included on both sides)."""
    rows, cols = 256, 512
    w = random_matrix(Q4_K, rows, cols, seed=3)
    x = np.random.default_rng(3).normal(0, 1, 300 * cols).astype(np.float32)
    W = gpu_ctx.upload(Q4_K, w, (cols, rows))
    full = W.matmul(x, 300).reshape(300, rows)
    for lo, hi in ((0, 129), (100, 300), (127, 257)):
        part = W.matmul(x[lo * cols:hi * cols], hi - lo).reshape(hi - lo, rows)
        assert np.array_equal(part, full[lo:hi]), (lo, hi)
    few = W.matmul(x[:128 * cols], 128).reshape(128, rows)
    for lo, hi in ((0, 2), (60, 128), (126, 128)):
        part = W.matmul(x[lo * cols:hi * cols], hi - lo).reshape(hi - lo, rows)
        assert np.array_equal(part, few[lo:hi]), (lo, hi)
    # both splits agree with each other to the f16 path's tolerance
    assert np.allclose(few, full[:128], rtol=0, atol=2e-3 * np.abs(full[:128]).max())


@pytest.mark.parametrize("dtype,rows,cols,batch", [(Q8_0, 2048, 2048, 64), (Q4_K, 2048, 2048, 16),
                                                   (Q2_0C, 1024, 4096, 5), (STQ1_0, 512, 2048, 128)],
                         ids=["q80_shared_64", "q4k_16", "q2c_5", "stq_128"])
def test_matmul_few_tokens_split_k(gpu_ctx, oracle, dtype, rows, cols, batch):
    """Batches of at most 128 tokens on weights of few row tiles run with K cut
    into up to 8 slices (Q8_0 in whole 256-column sets takes the one-launch
    register-operand product instead: the MoE shared projection [2048x2048]
    at 64 tokens); parity with the oracle as every batched product."""
    _print("gemm few tokens", NAMES[dtype], rows, cols, batch)
    w = random_matrix(dtype, rows, cols, seed=rows + batch)
    x = np.random.default_rng(batch).normal(0, 1, batch * cols).astype(np.float32)
    W = gpu_ctx.upload(dtype, w, (cols, rows))
    y = W.matmul(x, batch).reshape(batch, rows)
    y_ref, mag = oracle.matmul_f64(dtype, w, rows, cols, x, batch)
    check_prefill_path(y, y_ref, mag, f"{NAMES[dtype]} batch {batch}")
    W.release()


@pytest.mark.parametrize("rows,cols", [(1000, 256), (48, 768), (2048, 2048), (130, 4352)],
                         ids=["1000x256", "48x768", "2048x2048", "130x4352"])
def test_q80_few_tokens(gpu_ctx, oracle, rows, cols):
    """Q8_0 at 2..128 tokens (widths in 256-column sets) takes the one-launch
    register-operand product: parity with the oracle at 2, 17, 64 and 128
    tokens (one set, so that most waves have no share of K, and three sets,
    split unevenly; rows not a multiple of 16; two chunk groups), and every
    token's row bit-identical across those batches."""
    _print("q80 few tokens", rows, cols)
    w = random_matrix(Q8_0, rows, cols, seed=rows + cols)
    x = np.random.default_rng(cols).normal(0, 1, 128 * cols).astype(np.float32)
    W = gpu_ctx.upload(Q8_0, w, (cols, rows))
    full = W.matmul(x, 128).reshape(128, rows)
    y_ref, mag = oracle.matmul_f64(Q8_0, w, rows, cols, x, 128)
    check_prefill_path(full, y_ref, mag, f"Q8_0 {rows}x{cols} batch 128")
    for lo, hi in ((0, 2), (30, 47), (64, 128), (100, 101 + 27)):
        part = W.matmul(x[lo * cols:hi * cols], hi - lo).reshape(hi - lo, rows)
        assert np.array_equal(part, full[lo:hi]), (lo, hi)
    W.release()


def test_batched_rows_match_across_workgroup_forms(gpu_ctx):
    """96 row tiles at 300 tokens take the 8-wave, 256-token workgroups (a
    grid of 192); 2 and 50 tokens take the 4-wave, 128-token ones. Every
    element sees the same operands in the same order, so the rows agree bit
    for bit (a 256-token tile boundary and its partial tile included)."""
    rows, cols = 96 * 128, 256
    for dtype, seed in ((Q4_K, 11), (Q2_0C, 12)):
        ccols = 512 if dtype == Q2_0C else cols
        w = random_matrix(dtype, rows, ccols, seed=seed)
        x = np.random.default_rng(seed).normal(0, 1, 300 * ccols).astype(np.float32)
        W = gpu_ctx.upload(dtype, w, (ccols, rows))
        full = W.matmul(x, 300).reshape(300, rows)
        for lo, hi in ((0, 2), (255, 257), (250, 300)):
            part = W.matmul(x[lo * ccols:hi * ccols], hi - lo).reshape(hi - lo, rows)
            assert np.array_equal(part, full[lo:hi]), (NAMES[dtype], lo, hi)
        W.release()


def test_batched_shape_errors(gpu_ctx):
    W2 = gpu_ctx.upload(Q2_0C, random_matrix(Q2_0C, 8, 512, seed=0), (512, 8))
    with pytest.raises(ValueError):
        W2.matmul(np.zeros(3 * 512 - 1, np.float32), 3)


def test_activation_rows_scale_exactly(gpu_ctx):
    """Activations are rounded to f16 with a power-of-two scale per token row,
    so scaling a row by 2^k scales its output row by exactly 2^k, far beyond
    the f16 range (2^40) and below its normals (2^-40)."""
    rows, cols, batch = 160, 1024, 5
    w = random_matrix(Q6_K, rows, cols, seed=9)
    x = np.random.default_rng(9).normal(0, 1, (batch, cols)).astype(np.float32)
    W = gpu_ctx.upload(Q6_K, w, (cols, rows))
    base = W.matmul(x.reshape(-1), batch).reshape(batch, rows)
    k = np.array([40, -40, 0, 17, -3], np.float32)
    xs = (x * np.exp2(k)[:, None]).astype(np.float32)
    scaled = W.matmul(xs.reshape(-1), batch).reshape(batch, rows)
    assert np.array_equal(scaled, (base * np.exp2(k)[:, None]).astype(np.float32))
    zero = W.matmul(np.zeros(2 * cols, np.float32), 2)
    assert np.array_equal(zero, np.zeros(2 * rows, np.float32))


def test_f16_range_of_batched_weights(gpu_ctx):
    """The batched products round weights to f16: a tensor whose values could
    exceed f16's largest finite value, or whose values all lie below its
    smallest normal, is refused there (HYQ_EINVAL) while batch 1 (the int8
    GEMV, f32 arithmetic) still takes it."""
    from synth import set_block_scale
    rows, cols = 64, 512
    x = np.random.default_rng(4).normal(0, 1, 2 * cols).astype(np.float32)
    for d, ok in ((60000.0, False), (6e-8, False), (0.02, True)):
        w = set_block_scale(Q4_K, random_matrix(Q4_K, rows, cols, seed=5), d, dmin=d)
        W = gpu_ctx.upload(Q4_K, w, (cols, rows))
        assert np.all(np.isfinite(W.matmul(x[:cols], 1)))
        if ok:
            assert np.all(np.isfinite(W.matmul(x, 2)))
        else:
            with pytest.raises(ValueError, match="f16"):
                W.matmul(x, 2)
        W.release()
