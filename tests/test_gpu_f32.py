"""GPU parity of Weight::matmul by decoded rows (src/quant.rs:225-237 at
batch 1, :272-343 batched): F32 and F16 weights (the HyV3 router is F32,
src/model.rs:223-226) and Q8_0 widths that are whole 32-value blocks but not
whole 256-value groups, against the oracle's f64 products of the decoded
rows. Bar: the reference's own |err| <= 1e-5 * sum|w x| per element
(src/quant.rs:3021-3024) and 1e-4 relative in the 2-norm: these products are
f32 sums of exact f32 terms."""
import numpy as np
import pytest

from gpu_util import check_decode_path
from synth import F16, F32, Q8_0, random_matrix

pytestmark = pytest.mark.gpu

CASES = [(F32, 64, 2048), (F16, 1000, 1536), (F32, 37, 1001), (F16, 130, 6), (Q8_0, 300, 96),
         (Q8_0, 70, 2080)]


@pytest.mark.parametrize("dtype,rows,cols", CASES)
@pytest.mark.parametrize("batch", [1, 7, 130])
def test_decoded_row_matmul_matches_oracle(gpu_ctx, oracle, dtype, rows, cols, batch):
    w = random_matrix(dtype, rows, cols, seed=rows + cols)
    x = np.random.default_rng(batch).normal(0, 1, batch * cols).astype(np.float32)
    W = gpu_ctx.upload(dtype, w, (cols, rows))
    y = W.matmul(x, batch).reshape(batch, rows)
    y_ref, mag = oracle.matmul_f64(dtype, w, rows, cols, x, batch)
    for b in range(batch):
        check_decode_path(y[b], y_ref[b], mag[b], f"{dtype} [{rows}x{cols}] b{b}")
    # the reference's x86 arm (decoded row + AVX2-ordered dot) at batch 1
    if batch == 1:
        y_x86 = oracle.matmul(dtype, w, rows, cols, x, 1)
        assert np.allclose(y[0], y_x86[0], rtol=1e-5, atol=1e-5 * float(np.max(mag)))
    W.release()


def test_router_device_entry_point(gpu_ctx, hyq, oracle):
    """hyq_matmul_d on device buffers: the F32 router of 64 experts over a
    2048-wide hidden row, at batch 1 and batch 64."""
    rows, cols = 64, 2048
    w = random_matrix(F32, rows, cols, seed=3)
    W = gpu_ctx.upload(F32, w, (cols, rows))
    for batch in (1, 64):
        x = np.random.default_rng(batch).normal(0, 1, batch * cols).astype(np.float32)
        xd, yd = gpu_ctx.array(x), gpu_ctx.empty(batch * rows, np.float32)
        hyq.check(hyq.lib().hyq_matmul_d(gpu_ctx.handle, W.handle, xd.ptr, batch, yd.ptr))
        y_ref, mag = oracle.matmul_f64(F32, w, rows, cols, x, batch)
        y = yd.numpy().reshape(batch, rows)
        for b in range(batch):
            check_decode_path(y[b], y_ref[b], mag[b], f"router b{b}")


@pytest.mark.parametrize("dtype", [F32, F16])
def test_qkv_and_gate_up_of_decoded_rows(gpu_ctx, oracle, dtype):
    """gemv_qkv = three matmuls (src/quant.rs:716-720); matmul_gate_up_silu =
    two matmuls and silu(g) * u (:831-838)."""
    cols = 512
    ws = {n: random_matrix(dtype, r, cols, seed=i) for i, (n, r) in
          enumerate((("q", 256), ("k", 64), ("v", 64), ("g", 384), ("u", 384)))}
    W = {n: gpu_ctx.upload(dtype, a, (cols, a.size // cols // (2 if dtype == F16 else 4)))
         for n, a in ws.items()}
    x = np.random.default_rng(5).normal(0, 1, cols).astype(np.float32)
    yq, yk, yv = type(W["q"]).gemv_qkv(W["q"], W["k"], W["v"], x)
    for n, y in (("q", yq), ("k", yk), ("v", yv)):
        assert np.array_equal(y, W[n].matmul(x, 1)), n
    h = W["g"].matmul_gate_up_silu(W["u"], x)
    g, u = W["g"].matmul(x, 1), W["u"].matmul(x, 1)
    exp = (g / (np.float32(1.0) + np.exp(-g))) * u
    assert np.allclose(h, exp, rtol=2e-6, atol=1e-7)
