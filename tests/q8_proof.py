"""Accounting for int8 rounding flips in the decode-path parity tests.

Every batch-1 product quantizes its f32 input to int8 (Q8::quantize_into,
src/quant.rs:904-922). The device and the oracle form that input with f32
operations in different orders, so the two inputs can differ in their last
bits; where x * (127 / max) sits at a rounding midpoint (k + 0.5), such a
difference moves one int8 code by one, which changes the product by about
6e-4 of its norm. The device records, for every stage that quantizes (the
GEMV input stages, the RMSNorm+Q8 and quantize kernels), the f32 values it
quantized and the codes and scales it formed (hyq_ctx_set_q8_trace). These
helpers turn an output difference into a proof instead of an allowance:

  1. the oracle reruns the layer (or the output, or the MoE FFN) with the
     device's codes and scales in place of its own at every stage, recording
     its own f32 input of each stage;
  2. at every stage the device's codes and scales are the oracle quantizer's
     output on the device's own f32 input, bit for bit, and that input is
     within the decode bar (1e-4 relative) of the oracle's: any code where
     the two sides differ is then a rounding flip of inputs that agree to
     1e-4 (the two scaled values lie on either side of a k + 0.5 midpoint);
  3. with the device's codes, the outputs agree within the decode bar, with
     no exception.
"""
import numpy as np

import oracle as O

DECODE_BAR = 1e-4


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _scaled(x, s_codes):
    """x * (127 / max) per 256-group in f32, as the quantizer forms it."""
    g = x.reshape(-1, 256)
    m = np.abs(g).max(axis=1)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = np.where(m > 0, np.float32(127.0) / m.astype(np.float32), np.float32(0.0))
    return (g * inv.astype(np.float32)[:, None]).astype(np.float32).reshape(-1)


def explain_stage(x_own, q_own, s_own, q_dev, s_dev, x_dev, where):
    """The device's record of one stage against the oracle's f32 input of the
    same stage (steps 2 above). Returns the flips as (index, oracle code,
    device code, oracle's and device's distance to the midpoint)."""
    assert q_dev.size == q_own.size == x_dev.size and s_dev.size == s_own.size, where
    q_ref, s_ref = O.q8_quantize(x_dev)
    assert np.array_equal(q_dev, q_ref), (where, "device codes are not its input's")
    assert np.array_equal(s_dev.view(np.uint32), s_ref.view(np.uint32)), (where, "scales")
    r = rel(x_dev, x_own)
    assert r <= DECODE_BAR, (where, "stage input rel", r)
    d = q_dev.astype(np.int32) - q_own.astype(np.int32)
    idx = np.nonzero(d)[0]
    if idx.size == 0:
        return []
    assert np.all(np.abs(d[idx]) == 1), (where, "codes off by more than one", idx[:8])
    mid = (q_own[idx].astype(np.float64) + q_dev[idx].astype(np.float64)) / 2
    vo = _scaled(x_own, s_own)[idx].astype(np.float64)
    vd = _scaled(x_dev, s_dev)[idx].astype(np.float64)
    return [(int(i), int(q_own[i]), int(q_dev[i]), float(a), float(b))
            for i, a, b in zip(idx, np.abs(vo - mid), np.abs(vd - mid))]


def split_step_records(recs, ref, layers):
    """The device records of one decode step (hyq_dense_forward) as per-layer
    {stage: (codes, scales)} dicts in the oracle's stage numbering, plus the
    output's. A dense layer records its four input stages (QKV, attention
    output, gate/up, down); an MoE layer the first three, the shared down
    projection's and one record for all the routed experts' down inputs."""
    it = iter(recs)
    out = []
    for l in range(layers):
        widths = ref.stages(l)
        st = {}
        for k in range(4):
            q, s, x = next(it)
            assert q.size == widths[k], (l, k, q.size, widths[k])
            st[k] = (q, s, x)
        if len(widths) > 4:
            q, s, x = next(it)
            m, used = widths[4], len(widths) - 4
            assert q.size == m * used, (l, q.size, m, used)
            for j in range(used):
                st[4 + j] = (q[j * m:(j + 1) * m], s[j * m // 256:(j + 1) * m // 256],
                             x[j * m:(j + 1) * m])
        out.append(st)
    final = {0: next(it)}
    assert next(it, None) is None, "more records than the step's stages"
    return out, final


def prove(label, pairs, tap, stages, flips_seen, bar=DECODE_BAR):
    """Steps 2 and 3 for one oracle rerun on the device's codes: the flips
    of every stage are explained (and appended to flips_seen), then each
    (device, oracle) output pair agrees within the bar. Returns the largest
    relative error (0 without pairs)."""
    for st, (q, s, x) in sorted(stages.items()):
        x_o, q_o, s_o = tap.own(st, q.size)
        for f in explain_stage(x_o, q_o, s_o, q, s, x, (label, st)):
            flips_seen.append((label, st) + f)
    errs = [rel(a, b) for a, b in pairs]
    if errs:
        assert max(errs) <= bar, (label, errs)
    return max(errs, default=0.0)


def print_flips(label, flips):
    """One line per flip: where, stage, index, the two codes, and how far
    the oracle's and the device's scaled values were from their midpoint."""
    if not flips:
        print(label, "no int8 flips", flush=True)
    for where, st, i, own, dev, do, dd in flips:
        print(f"{label} flip: {where} stage {st} index {i} oracle {own} device {dev} "
              f"|x*inv - midpoint| oracle {do:.1e} device {dd:.1e}", flush=True)


def step_with_device_codes(ref, cfg, hidden, kcache, vcache, pos, layer_stages, final_stages,
                           label, flips_seen):
    """The oracle's own chain for one token (its own hidden rows and K/V
    rows, written to kcache/vcache at pos) with the device's codes at every
    stage: its logits. Each stage's flips are checked as above; the caller
    compares the logits."""
    h = hidden
    for l in range(cfg["layers"]):
        h, tap = ref.layer_tap(l, h, kcache[l], vcache[l], pos, use=layer_stages[l])
        prove((label, l), [], tap, layer_stages[l], flips_seen)
    logits, tap = ref.output_tap(h, use=final_stages)
    prove((label, "output"), [], tap, final_stages, flips_seen)
    return logits


def embed_row(model, cfg, token):
    rb = model["embed"].size // cfg["vocab"]
    return O.decode(model["embed_dtype"], model["embed"][token * rb:(token + 1) * rb])


def check_step(ctx, ref, model, cfg, kf, vf, pos, token, logits, nxt, label):
    """One traced decode step (ctx's record holds exactly that step's) against
    the oracle's own chain on caches kf/vf with the device's codes: every
    stage proved as above, the logits within the decode bar, and the same
    greedy token where the oracle's top-2 gap is clear. Returns the relative
    error of the logits."""
    stages, final = split_step_records(ctx.q8_trace(), ref, cfg["layers"])
    flips = []
    ref_logits = step_with_device_codes(ref, cfg, embed_row(model, cfg, token), kf, vf, pos,
                                        stages, final, label, flips)
    r = rel(logits, ref_logits)
    print(f"{label}: logits rel {r:.2e} on the device's codes "
          f"({len(flips)} flipped codes explained)", flush=True)
    assert r <= DECODE_BAR, (label, r)
    top = np.sort(ref_logits)[-2:]
    if top[1] - top[0] > 1e-3 * np.abs(ref_logits).max():
        assert nxt == int(np.argmax(ref_logits)), label
    return r
