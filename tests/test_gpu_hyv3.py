"""GPU parity of the HyV3 (MoE) arm against the oracle: route
(src/model.rs:728-767), Moe::forward (:687-726) as one device entry point at
batch 1 and batch n, and the decoder with MoE layers (forward_into's MoE call
site, :507-510 and :598-601) with the hy_v3 Q/K-norm order (:425-446).

Bars: expert selections equal; route weights within 2 f32 ulps (the GPU's
expf and glibc's differ by an ulp); a batch-1 MoE FFN within 1e-4 relative
on the device's int8 codes, every code where they differ from the oracle's
shown to be a rounding-midpoint flip (tests/q8_proof.py); an f16-MFMA batch
within 2e-3; decoder layers teacher-forced and free-running as in
test_gpu_c3.py."""
import numpy as np
import pytest

import q8_proof as P
from synth import Q4_K, Q8_0, make_hyv3_model, make_kv_cache, load_hyv3, upload_moe

TRACE_BYTES = 4 << 20

pytestmark = pytest.mark.gpu


def _print(*a):
    print(*a, flush=True)


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("experts,used,normalize", [(64, 8, True), (64, 8, False),
                                                    (160, 6, True), (7, 7, True),
                                                    (1024, 16, True)])
def test_route_matches_oracle(gpu_ctx, hyq, oracle, experts, used, normalize):
    tokens = 37
    rng = np.random.default_rng(experts + used)
    logits = rng.normal(0, 1, (tokens, experts)).astype(np.float32)
    bias = rng.normal(0, 0.1, experts).astype(np.float32)
    # ties: equal keys must fall back to the lower index
    logits[3, :] = 0.5
    bias_t = bias.copy()
    logits[4, :4] = [1.0, 1.0, -30.0, -31.0]  # tiny sigmoids, the floored sum
    pt, pe, pw = hyq.moe_route(gpu_ctx, logits, bias, used, normalize, 2.826)
    for t in range(tokens):
        ref = sorted(oracle.route(logits[t], bias_t, used, normalize, 2.826))
        sl = slice(t * used, (t + 1) * used)
        assert list(pt[sl]) == [t] * used
        assert list(pe[sl]) == [e for e, _ in ref], t
        w = np.array([v for _, v in ref], np.float32)
        assert np.allclose(pw[sl], w, rtol=3e-7, atol=0), (t, pw[sl], w)
    # all-equal logits and bias: the lowest indices, in order
    flat = np.zeros((1, experts), np.float32)
    _, pe, _ = hyq.moe_route(gpu_ctx, flat, np.zeros(experts, np.float32), used, normalize, 1.0)
    assert list(pe) == list(range(used))


MOE_C5 = dict(experts=64, used=8, mid=1536, shared_mid=1536, normalize=True, scale=2.5)
HYV3 = dict(layers=3, hidden=2048, heads=16, kv_heads=4, head_dim=128, ffn=6144, vocab=8192,
            rope_base=11158840.0, rms_eps=1e-5)


def _moe_model(moe, seed):
    return make_hyv3_model(dict(HYV3, layers=2), moe, linear=Q4_K, expert=Q4_K, shared=Q8_0,
                           seed=seed)


def test_moe_forward_one_token(gpu_ctx, hyq, oracle):
    """Moe::forward of single rows (the decode step's int8 GEMVs) at the
    30B-A3B-style shape: 64 Q4_K experts of width 1536, top 8, a Q8_0
    shared expert."""
    model = _moe_model(MOE_C5, seed=2)
    e = model["layers"][1]["moe"]
    H = HYV3["hidden"]
    ffn = upload_moe(hyq, gpu_ctx, e, H)
    gpu_ctx.set_q8_trace(TRACE_BYTES)
    errs, flips = [], []
    for s in range(4):
        x = np.random.default_rng(s).normal(0, 1, (1, H)).astype(np.float32)
        gpu_ctx.clear_q8_trace()
        got = ffn.forward(x)
        # the records: the row's Q8, the shared expert's down input, the
        # routed experts' down inputs (one record, slot after slot)
        rx, rs, (qe, se, xe) = gpu_ctx.q8_trace()
        m, used = e["mid"], e["used"]
        assert qe.size == m * used
        stages = {oracle.STAGE_FFN_IN: rx, oracle.STAGE_DOWN_IN: rs}
        for j in range(used):
            stages[oracle.STAGE_EXPERT_DOWN_IN + j] = (
                qe[j * m:(j + 1) * m], se[j * m // 256:(j + 1) * m // 256], xe[j * m:(j + 1) * m])
        ref, tap = oracle.moe_forward_tap(e, H, x, use=stages)
        errs.append(P.prove(f"moe row {s}", [(got, ref)], tap, stages, flips))
    gpu_ctx.set_q8_trace(None)
    _print("moe batch-1 rel on the GPU's codes", ["%.1e" % v for v in errs])
    P.print_flips("moe batch-1", flips)


@pytest.mark.parametrize("n", [5, 64])
def test_moe_forward_batch(gpu_ctx, hyq, oracle, n):
    """n rows: F32 router GEMM, route, the shared expert and the grouped
    expert kernels (f16 MFMA) against the oracle's f32 products."""
    moe = dict(MOE_C5, experts=32, mid=512, shared_mid=1024)
    model = _moe_model(moe, seed=3)
    e = model["layers"][1]["moe"]
    H = HYV3["hidden"]
    ffn = upload_moe(hyq, gpu_ctx, e, H)
    x = np.random.default_rng(n).normal(0, 1, (n, H)).astype(np.float32)
    got = ffn.forward(x)
    ref = oracle.moe_forward(e, H, x, n, int8_path=False)
    rel = _rel(got, ref)
    _print(f"moe batch {n} rel {rel:.2e}")
    assert rel <= 2e-3


def _teacher_forced(ref, dec, stages, final, cfg, pos, logits, label):
    """Each layer (dense or MoE) on the GPU's input row, cache and int8 codes,
    then the output: every flip explained, everything within 1e-4."""
    tr = dec.trace(1)[:, 0]
    errs, flips = [], []
    for l in range(cfg["layers"]):
        kc, vc = dec.read_kv(l, pos + 1)
        kref = np.zeros((pos + 1, kc.shape[1]), np.float32)
        vref = kref.copy()
        kref[:pos] = kc[:pos]
        vref[:pos] = vc[:pos]
        out, tap = ref.layer_tap(l, tr[l], kref, vref, pos, use=stages[l])
        errs.append(P.prove((label, l), [(tr[l + 1], out), (kc[pos], kref[pos]),
                                         (vc[pos], vref[pos])], tap, stages[l], flips))
    lg, tap = ref.output_tap(tr[-1], use=final)
    errs.append(P.prove((label, "output"), [(logits, lg)], tap, final, flips))
    _print(label, "per-layer rel on the GPU's codes (last: logits)",
           ["%.1e" % e for e in errs])
    P.print_flips(label, flips)


def test_hyv3_decoder_matches_oracle(gpu_ctx, hyq, oracle):
    """Three layers (a dense one, then two MoE layers of 64 experts) at the
    30B-A3B-style shapes, cache pre-filled to 700 of 768 positions; four
    tokens checked layer by layer and free-running; the graph replay of the
    same steps gives the same tokens."""
    cfg = HYV3
    context, prefilled = 768, 700
    model = make_hyv3_model(cfg, MOE_C5, linear=Q4_K, expert=Q4_K, shared=Q8_0, seed=4)
    dec = load_hyv3(hyq, gpu_ctx, model, context)
    k, v = make_kv_cache(cfg, context, prefilled, seed=4)
    for l in range(cfg["layers"]):
        dec.load_kv(l, k[l, :prefilled], v[l, :prefilled])
    dec.position = prefilled
    k0, v0 = k.copy(), v.copy()
    ref = oracle.DenseOracle(model)
    dec.set_trace(1)
    gpu_ctx.set_q8_trace(TRACE_BYTES)
    token, toks = 11, []
    for i in range(4):
        pos = prefilled + i
        gpu_ctx.clear_q8_trace()
        logits, nxt = dec.forward(token)
        stages, final = P.split_step_records(gpu_ctx.q8_trace(), ref, cfg["layers"])
        _teacher_forced(ref, dec, stages, final, cfg, pos, logits, f"hyv3 step {i}")
        # free-running: the oracle's own chain on the GPU's codes
        flips = []
        ref_logits = P.step_with_device_codes(ref, cfg, P.embed_row(model, cfg, token), k, v,
                                              pos, stages, final, f"hyv3 step {i}", flips)
        rel = P.rel(logits, ref_logits)
        _print(f"hyv3 step {i}: free-running logits rel {rel:.2e} on the GPU's codes "
               f"({len(flips)} flipped codes explained)")
        assert rel <= P.DECODE_BAR, (i, rel)
        top = np.sort(ref_logits)[-2:]
        if top[1] - top[0] > 1e-3 * np.abs(ref_logits).max():
            assert nxt == int(np.argmax(ref_logits))
        toks.append(nxt)
        token = nxt
    gpu_ctx.set_q8_trace(None)
    dec.set_trace(None)
    for l in range(cfg["layers"]):
        dec.load_kv(l, k0[l, :prefilled], v0[l, :prefilled])
    dec.position = prefilled
    assert list(dec.generate(11, 4, use_graph=True)) == toks
    dec.close()


def test_hyv3_prefill_matches_oracle(gpu_ctx, hyq, oracle):
    """hyq_dense_prefill of 120 tokens through a HyV3 model (32 experts of
    width 512, top 8): every layer's rows against the oracle's batch-n layer
    on the GPU's inputs (f16-MFMA bar), the logits at the decode bar."""
    cfg = dict(HYV3, vocab=4096)
    moe = dict(MOE_C5, experts=32, mid=512, shared_mid=1024)
    context, prefilled, n = 512, 40, 120
    model = make_hyv3_model(cfg, moe, linear=Q4_K, expert=Q4_K, shared=Q8_0, seed=5)
    dec = load_hyv3(hyq, gpu_ctx, model, context)
    k, v = make_kv_cache(cfg, context, prefilled, seed=5)
    for l in range(cfg["layers"]):
        dec.load_kv(l, k[l, :prefilled], v[l, :prefilled])
    dec.position = prefilled
    ref = oracle.DenseOracle(model)
    dec.set_trace(n)
    gpu_ctx.set_q8_trace(TRACE_BYTES)
    toks = np.random.default_rng(n).integers(0, cfg["vocab"], n).astype(np.int32)
    logits, _ = dec.prefill(toks)
    recs = gpu_ctx.q8_trace()
    gpu_ctx.set_q8_trace(None)
    tr = dec.trace(n)
    errs = []
    for l in range(cfg["layers"]):
        kc, vc = dec.read_kv(l, prefilled + n)
        kref = np.zeros((prefilled + n, kc.shape[1]), np.float32)
        vref = kref.copy()
        kref[:prefilled] = kc[:prefilled]
        vref[:prefilled] = vc[:prefilled]
        out = ref.prefill_layer(l, tr[l], kref, vref, prefilled).reshape(n, -1)
        errs.append(_rel(tr[l + 1], out))
        assert _rel(kc[prefilled:], kref[prefilled:]) <= 2e-3, (l, "K rows")
    # the logits: one batch-1 product of the GPU's final row on its codes
    assert len(recs) == 1, len(recs)
    flips = []
    lg, tap = ref.output_tap(tr[-1, -1], use={0: recs[0]})
    lerr = P.prove("hyv3 prefill output", [(logits, lg)], tap, {0: recs[0]}, flips)
    _print("hyv3 prefill per-layer rel", ["%.1e" % e for e in errs], "logits %.1e" % lerr)
    P.print_flips("hyv3 prefill output", flips)
    assert max(errs) <= 2e-3, errs
    dec.set_trace(None)
    dec.close()


def test_moe_entry_point_errors(gpu_ctx, hyq):
    """The argument checks of hyq_moe_route_d / hyq_moe_forward_d (the
    reference's ensure! arms of Model::from_gguf's MoE binding,
    src/model.rs:206-235, and route's preconditions): each returns an error
    before any launch, and a valid call afterwards still runs."""
    import ctypes
    L = hyq.lib()
    moe = dict(MOE_C5, experts=8, used=2, mid=256, shared_mid=256)
    model = _moe_model(moe, seed=9)
    e = model["layers"][1]["moe"]
    H = HYV3["hidden"]
    ffn = upload_moe(hyq, gpu_ctx, e, H)
    r, g, u, d, sg, su, sd = ffn.weights
    x = gpu_ctx.array(np.random.default_rng(1).normal(0, 1, (3, H)).astype(np.float32))
    out = gpu_ctx.empty(3 * H, np.float32)
    need = L.hyq_moe_forward_scratch_bytes(ctypes.byref(ffn.cfg), H, 3)
    assert need > 0
    scratch = gpu_ctx.empty(need, np.uint8)

    def fwd(cfg=None, router=r, gate=g, down=d, tokens=3, nbytes=need, xptr=None):
        return L.hyq_moe_forward_d(gpu_ctx.handle, ctypes.byref(cfg or ffn.cfg), router.handle,
                                   ffn.bias.ptr, gate.handle, u.handle, down.handle, sg.handle,
                                   su.handle, sd.handle, x.ptr if xptr is None else xptr, tokens,
                                   scratch.ptr, nbytes, out.ptr)
    EINVAL = hyq.EINVAL
    assert fwd(router=g) == EINVAL                               # not [hidden, experts]
    assert fwd(gate=d) == EINVAL                                 # gate shaped like down
    assert fwd(down=g) == EINVAL
    assert fwd(nbytes=need - 1) == EINVAL                        # scratch too small
    assert fwd(xptr=x.ptr + 4) == EINVAL                         # misaligned rows
    bad = hyq.MoeConfig(8, 9, 256, 256, 1, 2.5)                  # used > experts
    assert fwd(cfg=bad) == EINVAL
    bad = hyq.MoeConfig(8, 2, 256, 256, 1, 0.0)                  # non-positive scale
    assert fwd(cfg=bad) == EINVAL
    assert L.hyq_moe_forward_scratch_bytes(ctypes.byref(hyq.MoeConfig(8, 2, -1, 256, 1, 1.0)),
                                           H, 3) == 0
    # route: used > experts, too many experts, null buffers
    lg = gpu_ctx.array(np.zeros((2, 8), np.float32))
    bias = gpu_ctx.array(np.zeros(8, np.float32))
    pe = gpu_ctx.empty(2 * 2, np.int32)
    pw = gpu_ctx.empty(2 * 2, np.float32)
    f = ctypes.c_float(1.0)
    assert L.hyq_moe_route_d(gpu_ctx.handle, lg.ptr, bias.ptr, 2, 8, 9, 1, f, None, pe.ptr,
                             pw.ptr) == EINVAL
    assert L.hyq_moe_route_d(gpu_ctx.handle, lg.ptr, bias.ptr, 2, 2048, 2, 1, f, None, pe.ptr,
                             pw.ptr) == EINVAL
    assert L.hyq_moe_route_d(gpu_ctx.handle, lg.ptr, bias.ptr, 2, 8, 2, 1, f, None, None,
                             pw.ptr) == EINVAL
    # a valid call still runs and matches the Python wrapper's
    hyq.check(fwd())
    gpu_ctx.sync()
    assert np.array_equal(out.numpy().reshape(3, H), ffn.forward(x.numpy().reshape(3, H)))
