"""GPU tests of loading from GGUF (hyq_gguf_upload, hyq_gguf_read_f32,
hyq_dense_from_gguf: Gguf::tensor and Model::from_gguf, src/gguf.rs:212-218,
src/model.rs:136-262): a device weight uploaded from a file equals the one
uploaded from the same bytes directly, and a dense decoder loaded from a
file decodes bit-identically to one assembled by hand from the same model."""
import numpy as np
import pytest

from gguf_writer import STR, U32, build, dense_model_file
from synth import Q2_0C, Q4_K, Q6_K, STQ1_0, load_dense, make_dense_model, random_matrix

pytestmark = pytest.mark.gpu

SMALL = dict(layers=2, hidden=512, heads=4, kv_heads=1, head_dim=128, ffn=1024, vocab=3000,
             rope_base=11158840.0, rms_eps=1e-5)


def _print(*a):
    print(*a, flush=True)


def test_upload_and_read_from_a_standard_file(gpu_ctx, hyq, tmp_path):
    rows, cols = 384, 1024
    w = random_matrix(Q4_K, rows, cols, seed=12)
    norm = np.random.default_rng(1).normal(1, 0.02, cols).astype(np.float32)
    path = tmp_path / "m.gguf"
    path.write_bytes(build([("general.architecture", STR, "x")],
                           [("w", [cols, rows], 12, w.tobytes()), ("n", [cols], 0, norm.tobytes())]))
    g = hyq.Gguf(str(path))
    assert g.profile == "standard"
    Wg = g.upload(gpu_ctx, "w")
    Wd = gpu_ctx.upload(Q4_K, w, (cols, rows))
    assert Wg.shape() == (cols, rows) and Wg.dtype == Q4_K
    x = np.random.default_rng(2).normal(0, 1, (3, cols)).astype(np.float32)
    for b in (1, 3):
        a, d = Wg.matmul(x[:b].ravel(), b), Wd.matmul(x[:b].ravel(), b)
        assert np.array_equal(a.view(np.uint32), d.view(np.uint32))
    assert np.array_equal(g.read_f32(gpu_ctx, "n").view(np.uint32), norm.view(np.uint32))
    with pytest.raises(ValueError):
        g.upload(gpu_ctx, "n")  # a vector is not a matrix
    with pytest.raises(ValueError):
        g.upload(gpu_ctx, "missing")
    Wg.release()
    Wd.release()
    g.close()


@pytest.mark.parametrize("linear,tid,ft,profile", [(Q2_0C, 40, 39, "tencent-q2-0c"),
                                                   (STQ1_0, 42, 41, "tencent-stq1")])
def test_dense_decoder_from_gguf_equals_manual_load(gpu_ctx, hyq, tmp_path, linear, tid, ft,
                                                    profile):
    c = SMALL
    model = make_dense_model(c, linear=linear, seed=21)
    model["output"] = random_matrix(Q6_K, c["vocab"], c["hidden"], 71)
    path = tmp_path / "dense.gguf"
    path.write_bytes(dense_model_file(model, tid, file_type=ft))
    g = hyq.Gguf(str(path), profile=profile)
    assert g.profile == profile
    context = 64
    a = hyq.DenseDecoder.from_gguf(gpu_ctx, g, context)
    b = load_dense(hyq, gpu_ctx, model, context)
    tokens = np.random.default_rng(3).integers(0, c["vocab"], 20).astype(np.int32)
    la, ta = a.prefill(tokens)
    lb, tb = b.prefill(tokens)
    assert ta == tb and np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    sa, sb = a.generate(ta, 6), b.generate(tb, 6)
    assert np.array_equal(sa, sb)
    _print("from_gguf", profile, "tokens", sa)
    a.close()
    b.close()
    g.close()


def test_dense_from_gguf_errors(gpu_ctx, hyq, tmp_path):
    c = SMALL
    model = make_dense_model(c, linear=Q2_0C, seed=22)
    g = hyq.Gguf(data=dense_model_file(model, 40, file_type=39, context_length=32),
                 profile="tencent-q2-0c")
    with pytest.raises(ValueError, match="context must be"):
        hyq.DenseDecoder.from_gguf(gpu_ctx, g, 33)
    bad = dense_model_file(model, 40, file_type=39).replace(b"blk.1.ffn_down.weight",
                                                            b"blk.1.ffn_dowX.weight")
    with pytest.raises(ValueError, match="missing tensor blk.1.ffn_down.weight"):
        hyq.DenseDecoder.from_gguf(gpu_ctx, hyq.Gguf(data=bad, profile="tencent-q2-0c"), 8)
    other = build([("general.architecture", STR, "llama"), ("llama.block_count", U32, 1)], [])
    with pytest.raises(ValueError, match="unsupported model architecture llama"):
        hyq.DenseDecoder.from_gguf(gpu_ctx, hyq.Gguf(data=other), 8)


HYV3_SMALL = dict(layers=3, hidden=512, heads=4, kv_heads=1, head_dim=128, ffn=1024, vocab=3000,
                  rope_base=11158840.0, rms_eps=1e-5)
MOE_SMALL = dict(experts=16, used=4, mid=512, shared_mid=768, normalize=True, scale=2.5)


def test_hyv3_decoder_from_gguf_equals_manual_load(gpu_ctx, hyq, tmp_path):
    """Model::from_gguf's hy_v3 arm (src/model.rs:136-262): a dense first
    layer, MoE layers after it, a separate output; prefill and decoding
    bit-identical to the decoder assembled by hand from the same model."""
    from gguf_writer import hyv3_model_file
    from synth import Q8_0, load_hyv3, make_hyv3_model
    model = make_hyv3_model(HYV3_SMALL, MOE_SMALL, linear=Q4_K, expert=Q4_K, shared=Q8_0,
                            seed=23)
    path = tmp_path / "hyv3.gguf"
    path.write_bytes(hyv3_model_file(model))
    g = hyq.Gguf(str(path))
    context = 64
    a = hyq.DenseDecoder.from_gguf(gpu_ctx, g, context)
    b = load_hyv3(hyq, gpu_ctx, model, context)
    tokens = np.random.default_rng(4).integers(0, HYV3_SMALL["vocab"], 20).astype(np.int32)
    la, ta = a.prefill(tokens)
    lb, tb = b.prefill(tokens)
    assert ta == tb and np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    sa, sb = a.generate(ta, 6), b.generate(tb, 6)
    assert np.array_equal(sa, sb)
    _print("hy_v3 from_gguf tokens", sa)
    a.close()
    b.close()
    g.close()


@pytest.mark.parametrize("case,match", [
    ("gating", "sigmoid router"), ("no_output", "separate output"),
    ("no_bias", "missing tensor blk.1.exp_probs_b"), ("f16_router", "router must use F32")])
def test_hyv3_from_gguf_errors(gpu_ctx, hyq, case, match):
    """The hy_v3 arm's ensure! rules (src/model.rs:199-226)."""
    from gguf_writer import hyv3_model_file
    from synth import Q8_0, make_hyv3_model
    model = make_hyv3_model(dict(HYV3_SMALL, layers=2), MOE_SMALL, linear=Q4_K, expert=Q4_K,
                            shared=Q8_0, seed=24)
    if case == "gating":
        data = hyv3_model_file(model, gating=1)
    elif case == "no_output":
        data = hyv3_model_file(model, drop="output.weight")
    elif case == "no_bias":
        data = hyv3_model_file(model, drop="blk.1.exp_probs_b")
    else:
        data = hyv3_model_file(model, router_f16=True)
    with pytest.raises(ValueError, match=match):
        hyq.DenseDecoder.from_gguf(gpu_ctx, hyq.Gguf(data=data), 16)
