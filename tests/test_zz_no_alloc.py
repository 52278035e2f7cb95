"""hyq_matmul_noalloc_d: Weight::matmul on device buffers with every
temporary in the library's fixed per-device array (no device allocation).
Its results must equal hyq_matmul_d's bit for bit (same kernels, same K
slicing), on consecutive calls that reuse the array with a smaller input
second; a product whose temporaries exceed the array is rejected before any
work."""
import numpy as np
import pytest

from synth import F32, Q2_0C, Q4_K, Q6_K, Q8_0, random_matrix

pytestmark = pytest.mark.gpu

MAX_BYTES = 32 * 1024 * 1024


def _run(hyq, ctx, W, x, batch, rows, misalign=False):
    """(hyq_matmul_d, hyq_matmul_noalloc_d) outputs for the same input; with
    misalign the input starts 4 bytes past a 16-byte boundary, which sends a
    batch-1 product through a separate Q8 pass (the array holds its Q8 row)."""
    L = hyq.lib()
    buf = np.zeros(x.size + 4, np.float32)
    off = 1 if misalign else 0
    buf[off:off + x.size] = x
    xd = ctx.array(buf)
    xp = xd.ptr + 4 * off
    outs = []
    for fn in (L.hyq_matmul_d, L.hyq_matmul_noalloc_d):
        yd = ctx.empty(batch * rows, np.float32)
        hyq.check(fn(ctx.handle, W.handle, xp, batch, yd.ptr))
        outs.append(yd.numpy())
    return outs


CASES = [
    # (dtype, rows, cols, first batch, second (smaller) batch, misaligned batch-1 input)
    (Q8_0, 2048, 2048, 64, 5, False),    # 8 K slices: f16 rows + 4 MiB of partials
    (Q4_K, 6144, 2048, 130, 2, False),   # one K slice, 8-wave tiles
    (Q2_0C, 3072, 2048, 1, 1, True),     # batch 1, Q8 row in the array
    (Q6_K, 4096, 1024, 96, 1, True),     # batched, then a misaligned batch-1 row
    (F32, 64, 2048, 64, 1, False),       # decoded rows: no temporaries
]


@pytest.mark.parametrize("dtype,rows,cols,b1,b2,mis", CASES)
def test_noalloc_equals_matmul_d_twice(gpu_ctx, hyq, dtype, rows, cols, b1, b2, mis):
    w = random_matrix(dtype, rows, cols, seed=rows + b1)
    W = gpu_ctx.upload(dtype, w, (cols, rows))
    rng = np.random.default_rng(b1 * 7 + b2)
    for batch in (b1, b2):
        x = rng.normal(0, 1, batch * cols).astype(np.float32)
        ref, got = _run(hyq, gpu_ctx, W, x, batch, rows, misalign=mis and batch == 1)
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), (dtype, batch)
        assert np.all(np.isfinite(got))
    W.release()


def test_noalloc_rejects_oversized_products(gpu_ctx, hyq):
    """[14336 x 4096] Q4_K at 4096 tokens needs 32 MiB of f16 rows plus their
    scales: past the array, so HYQ_EINVAL and no launch; the same weight at
    64 tokens fits and matches hyq_matmul_d."""
    rows, cols = 14336, 4096
    assert 4096 * cols * 2 + 4096 * 4 > MAX_BYTES
    w = random_matrix(Q4_K, rows, cols, seed=2)
    W = gpu_ctx.upload(Q4_K, w, (cols, rows))
    xd = gpu_ctx.empty(4096 * cols, np.float32)
    yd = gpu_ctx.empty(4096 * rows, np.float32)
    with pytest.raises(ValueError, match="scratch"):
        hyq.check(hyq.lib().hyq_matmul_noalloc_d(gpu_ctx.handle, W.handle, xd.ptr, 4096, yd.ptr))
    x = np.random.default_rng(3).normal(0, 1, 64 * cols).astype(np.float32)
    ref, got = _run(hyq, gpu_ctx, W, x, 64, rows)
    assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))
    W.release()
