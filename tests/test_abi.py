"""CPU tests of the C ABI library: it loads, exports every symbol that
include/hyq.h declares, and rejects bad arguments before touching a device."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hyq.h")


@pytest.fixture(scope="module")
def lib(hyq):
    if not os.path.exists(hyq.LIB_PATH):
        import importlib.util
        spec = importlib.util.spec_from_file_location(
            "hyq_build", os.path.join(ROOT, "hy-mt-rs_amd", "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return hyq.lib()


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hyq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("hyq_matmul", "hyq_gemv_qkv", "hyq_gate_up_silu", "hyq_weight_expert",
                     "hyq_decode", "hyq_quantize_q8_d", "hyq_gemv_q8_d", "hyq_last_error"):
        assert required in names


def test_every_declared_symbol_is_exported(lib, hyq):
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in hyq.SIGNATURES, f"{name} has no ctypes signature"


def test_geometry(lib):
    expect = {0: (1, 4), 1: (1, 2), 8: (32, 34), 12: (256, 144), 14: (256, 210),
              40: (512, 130), 42: (256, 42)}
    for dt, (bl, bb) in expect.items():
        assert (lib.hyq_block_len(dt), lib.hyq_block_bytes(dt)) == (bl, bb)
    assert lib.hyq_block_len(2) == -1 and lib.hyq_block_bytes(43) == -1


def test_isums_per_row(lib):
    assert lib.hyq_isums_per_row(40, 2048) == 8
    assert lib.hyq_isums_per_row(42, 2048) == 8
    assert lib.hyq_isums_per_row(14, 2048) == 128
    assert lib.hyq_isums_per_row(12, 2048) == 16
    assert lib.hyq_isums_per_row(8, 2048) == 64
    assert lib.hyq_isums_per_row(0, 2048) == -1
    assert lib.hyq_isums_per_row(40, 300) == -1


def test_null_arguments_are_rejected_without_a_device(lib, hyq):
    out = ctypes.c_void_p()
    dims = (ctypes.c_uint64 * 3)(512, 8, 1)
    assert lib.hyq_weight_upload(None, 40, None, 0, ctypes.cast(dims, ctypes.c_void_p), 2,
                                 ctypes.byref(out)) == hyq.EINVAL
    assert b"null" in lib.hyq_last_error()
    assert lib.hyq_weight_expert(None, 0, ctypes.byref(out)) == hyq.EINVAL
    assert lib.hyq_matmul(None, None, None, 1, None) == hyq.EINVAL
    assert lib.hyq_gemv_q8_d(None, None, None, None, None) == hyq.EINVAL
    assert lib.hyq_sync(None) == hyq.EINVAL
    assert lib.hyq_decode(None, 40, None, 0, None, 0) == hyq.EINVAL
    assert lib.hyq_weight_info(None, None, None, None) == hyq.EINVAL
    lib.hyq_weight_release(None)
    lib.hyq_q8_release(None)
    lib.hyq_ctx_destroy(None)


def test_product_has_no_cpu_fallback(hyq):
    """The package computes only through libhyq.so: it never imports the oracle."""
    pkg = os.path.join(ROOT, "hy-mt-rs_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "libhyq_oracle" not in text and "import oracle" not in text, f
                assert "hyq_oracle" not in text, f
