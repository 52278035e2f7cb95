"""Helpers for GPU tests. Device buffers come from libhyq's own C ABI
(hyq_device_alloc / hyq_memcpy_*): the torch wheel bundles a second HIP/HSA
runtime that cannot share the device with libhyq's in one process, so GPU
tests never initialise torch's GPU backend."""
from __future__ import annotations

import numpy as np


def check_decode_path(y: np.ndarray, y_ref: np.ndarray, mag: np.ndarray, label: str = ""):
    """Decode-path tolerance: the reference's own bound |err| <= 1e-5 * sum|terms|
    (src/quant.rs:3021-3024) per element, and 1e-4 relative in the 2-norm."""
    y = y.astype(np.float64)
    err = np.abs(y - y_ref)
    worst = int(np.argmax(err - 1e-5 * mag))
    assert np.all(err <= 1e-5 * mag), (
        f"{label}: row {worst} err {err[worst]:.3e} > 1e-5*mag {1e-5 * mag[worst]:.3e}")
    rel = np.linalg.norm(y - y_ref) / max(np.linalg.norm(y_ref), 1e-30)
    assert rel <= 1e-4, f"{label}: relative 2-norm error {rel:.3e}"
    return rel


def device_bytes(hyq, ctx, ptr: int, nbytes: int) -> np.ndarray:
    """Copy nbytes at a device address to the host."""
    out = np.empty(nbytes, np.uint8)
    hyq.check(hyq.lib().hyq_memcpy_d2h(ctx.handle, out.ctypes.data, ptr, nbytes))
    return out


def check_prefill_path(y: np.ndarray, y_ref: np.ndarray, mag: np.ndarray, label: str = ""):
    """f16-MFMA tolerance: per element |err| <= 2e-3 * sum|w x| and 2e-3
    relative in the 2-norm."""
    y = np.asarray(y, np.float64)
    err = np.abs(y - y_ref)
    bad = err > 2e-3 * mag
    assert not np.any(bad), (
        f"{label}: {int(bad.sum())} elements exceed 2e-3*mag; worst "
        f"{float(np.max(err / np.maximum(mag, 1e-30))):.3e}")
    rel = np.linalg.norm(y - y_ref) / max(np.linalg.norm(y_ref), 1e-30)
    assert rel <= 2e-3, f"{label}: relative 2-norm error {rel:.3e}"
    return rel
