"""The measurement aids bench.py compares the kernels with (no counterpart in
the reference): the read-only HBM stream reads every byte of its buffer once,
and the MFMA stream runs and rejects bad arguments."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_hbm_read_covers_the_buffer(gpu_ctx, hyq):
    """A buffer of ones: the per-workgroup sums add up to its float count
    (every 16-byte word read exactly once, the tail loop included)."""
    L = hyq.lib()
    for n_floats, wgs in ((1 << 20, 64), ((1 << 20) + 12, 37), (4, 1)):
        buf = gpu_ctx.array(np.ones(n_floats, np.float32))
        sink = gpu_ctx.empty(wgs, np.float32)
        hyq.check(L.hyq_hbm_read_d(gpu_ctx.handle, buf.ptr, n_floats * 4, wgs, sink.ptr))
        assert float(sink.numpy().astype(np.float64).sum()) == n_floats


def test_mfma_stream_runs_and_checks_arguments(gpu_ctx, hyq):
    L = hyq.lib()
    wgs, iters = 16, 8
    sink = gpu_ctx.empty(wgs * 256, np.float32)
    hyq.check(L.hyq_mfma_stream_d(gpu_ctx.handle, wgs, iters, sink.ptr))
    s = sink.numpy()
    assert np.all(np.isfinite(s)) and np.any(s != 0)
    # every workgroup computes the same values
    assert np.array_equal(s[:256], s[256:512])
    for bad in ((0, iters), (wgs, 0), (-1, iters)):
        assert L.hyq_mfma_stream_d(gpu_ctx.handle, bad[0], bad[1], sink.ptr) != 0
    assert L.hyq_mfma_stream_d(gpu_ctx.handle, wgs, iters, None) != 0
