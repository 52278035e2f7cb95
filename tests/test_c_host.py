"""The C ABI from a compiled C host (tests/c_host/hyq_host.c): include/hyq.h
as plain C11 (-pedantic -Werror), libhyq.so linked the way the reference's
Rust FFI shim would link it, and on the GPU Weight::matmul at batch 1 (int8
GEMV, host pointers) and at batch 64 (device buffers) checked against the
oracle inside that program, plus its error path."""
import os
import subprocess

import numpy as np
import pytest

from synth import NAMES, Q2_0C, Q4_K, Q6_K, STQ1_0, random_matrix

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST_DIR = os.path.join(ROOT, "tests", "c_host")
HOST = os.path.join(HOST_DIR, "hyq_host")


def test_header_builds_as_c_and_links(tmp_path):
    """Compiled here into a scratch directory: the header is valid C11, the
    program links against the built library, and without a device the
    context request fails with a code and a message."""
    exe = tmp_path / "hyq_host"
    cmd = ["gcc", "-O1", "-std=c11", "-Wall", "-Wextra", "-Werror", "-pedantic",
           f"-I{ROOT}/include", f"-I{ROOT}/oracle", "-o", str(exe),
           os.path.join(HOST_DIR, "hyq_host.c"),
           f"-L{ROOT}/hy-mt-rs_amd", "-lhyq", f"-L{ROOT}/oracle", "-lhyq_oracle", "-lm",
           f"-Wl,-rpath,{ROOT}/hy-mt-rs_amd", f"-Wl,-rpath,{ROOT}/oracle"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe), "--no-gpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "no device: code -3" in r.stdout or "device present" in r.stdout, r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [Q4_K, Q2_0C, STQ1_0, Q6_K], ids=lambda d: NAMES[d])
def test_c_host_matmul_on_gpu(tmp_path, dtype):
    assert os.path.exists(HOST), "tests/c_host/hyq_host is built by __graft_entry__.build()"
    rows, cols, batch = 200, 1024, 64
    w = random_matrix(dtype, rows, cols, seed=60 + dtype)
    path = tmp_path / "w.bin"
    np.asarray(w, np.uint8).tofile(path)
    print("c host", NAMES[dtype], rows, cols, batch, flush=True)
    r = subprocess.run([HOST, str(dtype), str(rows), str(cols), str(path), str(batch)],
                       capture_output=True, text=True, timeout=120)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("ok")
