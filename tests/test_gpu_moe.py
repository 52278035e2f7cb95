"""GPU parity of the MoE expert products (the expert loop of Moe::forward,
src/model.rs:699-725) through the C ABI.

The oracle is a float64 chain per routed pair built from the oracle's
row-local f64 products (gate and up in f64, silu(g)*u rounded to f32 as the
reference stores it, down in f64 over that f32 vector), summed per token in
ascending expert order onto the seed; oracle.moe_experts (the reference's
x86 f32 path restated) is checked against the same chain. Tolerance of the
f16-MFMA path: 2e-3 relative in the 2-norm, and per element
|err| <= 5e-3 * sum_p |w_p| * sum_k |down_e[i,k] h_k| (h carries the f16
errors of two products and its own f16 rounding)."""
import numpy as np
import pytest

from synth import NAMES, Q4_K, Q6_K, Q8_0, Q2_0C, STQ1_0, random_matrix, row_bytes

pytestmark = pytest.mark.gpu


def _print(*a):
    print(*a, flush=True)


def softmax_top(logits: np.ndarray, k: int):
    """Top-k of softmax(logits) (index tie-break), weights renormalized to sum 1."""
    z = logits.astype(np.float64) - logits.max()
    p = np.exp(z) / np.exp(z).sum()
    idx = sorted(range(len(p)), key=lambda i: (-p[i], i))[:k]
    w = p[idx] / p[idx].sum()
    return idx, w.astype(np.float32)


def routed_pairs(tokens, experts, used, seed):
    rng = np.random.default_rng(seed)
    pt, pe, pw = [], [], []
    for t in range(tokens):
        idx, w = softmax_top(rng.normal(0, 1, experts).astype(np.float32), used)
        pt += [t] * used
        pe += idx
        pw += list(w)
    return (np.array(pt, np.int32), np.array(pe, np.int32), np.array(pw, np.float32))


def chain_f64(oracle, fg, fd, gate, up, down, hidden, mid, x, pt, pe, pw, seed_out, tokens_of):
    """f64 reference of out[t] for t in tokens_of, plus its magnitude bound."""
    gb, db = row_bytes(fg, hidden) * mid, row_bytes(fd, mid) * hidden
    out = {t: seed_out[t].astype(np.float64).copy() for t in tokens_of}
    mag = {t: np.zeros(hidden) for t in tokens_of}
    order = sorted(range(len(pt)), key=lambda p: (pe[p], p))
    for p in order:
        t, e, w = int(pt[p]), int(pe[p]), float(pw[p])
        if t not in out:
            continue
        xt = x[t * hidden:(t + 1) * hidden]
        g, _ = oracle.matmul_f64(fg, gate[e * gb:(e + 1) * gb], mid, hidden, xt, 1)
        u, _ = oracle.matmul_f64(fg, up[e * gb:(e + 1) * gb], mid, hidden, xt, 1)
        with np.errstate(over="ignore"):
            h = (g[0] / (1 + np.exp(-g[0])) * u[0]).astype(np.float32)
        d, dm = oracle.matmul_f64(fd, down[e * db:(e + 1) * db], hidden, mid, h, 1)
        out[t] += np.float64(np.float32(w)) * d[0]
        mag[t] += abs(w) * dm[0]
    return out, mag


def check_moe(got, ref, mag, label):
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= 5e-3 * mag + 1e-6), (
        f"{label}: worst err/mag {float(np.max(err / np.maximum(mag, 1e-30))):.3e}")
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert rel <= 2e-3, f"{label}: relative 2-norm error {rel:.3e}"


@pytest.mark.parametrize("fg,fd", [(Q4_K, Q4_K), (Q4_K, Q6_K), (Q8_0, Q8_0), (Q2_0C, Q2_0C),
                                   (STQ1_0, STQ1_0)],
                         ids=lambda f: NAMES[f])
def test_moe_small_matches_chain(gpu_ctx, hyq, oracle, fg, fd):
    hidden, mid, experts, tokens, used = 512, 512, 8, 21, 3
    _print("moe", NAMES[fg], NAMES[fd])
    gate = random_matrix(fg, experts * mid, hidden, seed=1)
    up = random_matrix(fg, experts * mid, hidden, seed=2)
    down = random_matrix(fd, experts * hidden, mid, seed=3)
    x = np.random.default_rng(4).normal(0, 1, tokens * hidden).astype(np.float32)
    seed_out = np.random.default_rng(5).normal(0, 1, (tokens, hidden)).astype(np.float32)
    pt, pe, pw = routed_pairs(tokens, experts, used, seed=6)
    G = gpu_ctx.upload(fg, gate, (hidden, mid, experts))
    U = gpu_ctx.upload(fg, up, (hidden, mid, experts))
    D = gpu_ctx.upload(fd, down, (mid, hidden, experts))
    got = hyq.moe_experts(G, U, D, x, tokens, pt, pe, pw, seed_out).reshape(tokens, hidden)
    ref, mag = chain_f64(oracle, fg, fd, gate, up, down, hidden, mid, x, pt, pe, pw, seed_out,
                         range(tokens))
    R = np.stack([ref[t] for t in range(tokens)])
    M = np.stack([mag[t] for t in range(tokens)])
    check_moe(got, R, M, f"{NAMES[fg]}/{NAMES[fd]}")
    if fg == fd:
        # the reference's own x86 f32 path agrees with the f64 chain
        cpu = oracle.moe_experts(fg, fd, gate, up, down, experts, hidden, mid, x, pt, pe, pw,
                                 seed_out.reshape(-1), threads=4).reshape(tokens, hidden)
        assert np.all(np.abs(cpu - R) <= 1e-4 * M + 1e-6)


def test_moe_uneven_groups_and_empty_experts(gpu_ctx, hyq, oracle):
    """One expert with 150 tokens (two 128-token chunks), several empty
    experts, a token routed to no expert, pairs not grouped by token."""
    hidden, mid, experts, tokens = 256, 768, 6, 160
    gate = random_matrix(Q4_K, experts * mid, hidden, seed=11)
    up = random_matrix(Q4_K, experts * mid, hidden, seed=12)
    down = random_matrix(Q4_K, experts * hidden, mid, seed=13)
    x = np.random.default_rng(14).normal(0, 1, tokens * hidden).astype(np.float32)
    seed_out = np.zeros((tokens, hidden), np.float32)
    pt = [t for t in range(150)] + [3, 7, 159, 3]
    pe = [2] * 150 + [5, 5, 0, 0]
    pw = list(np.random.default_rng(15).uniform(0.1, 1.0, len(pt)))
    pt, pe, pw = np.array(pt, np.int32), np.array(pe, np.int32), np.array(pw, np.float32)
    perm = np.random.default_rng(16).permutation(len(pt))
    pt, pe, pw = pt[perm], pe[perm], pw[perm]
    G = gpu_ctx.upload(Q4_K, gate, (hidden, mid, experts))
    U = gpu_ctx.upload(Q4_K, up, (hidden, mid, experts))
    D = gpu_ctx.upload(Q4_K, down, (mid, hidden, experts))
    got = hyq.moe_experts(G, U, D, x, tokens, pt, pe, pw, seed_out).reshape(tokens, hidden)
    ref, mag = chain_f64(oracle, Q4_K, Q4_K, gate, up, down, hidden, mid, x, pt, pe, pw,
                         seed_out, range(tokens))
    R = np.stack([ref[t] for t in range(tokens)])
    M = np.stack([mag[t] for t in range(tokens)])
    check_moe(got, R, M, "uneven")
    assert np.all(got[150:159] == 0.0)  # tokens 150..158 are routed nowhere


def test_moe_q4k_few_token_chunks(gpu_ctx, hyq, oracle):
    """Pairs averaging at most 16 per expert take the Q4_K register kernels:
    one expert with 40 tokens (16-token chunks 16 + 16 + 8), empty experts, a
    token routed nowhere, and token rows scaled by 1e6 and 1e-6 (the f16 row
    scale of the activation operand and of the SiLU product)."""
    hidden, mid, experts, tokens = 512, 768, 12, 44
    gate = random_matrix(Q4_K, experts * mid, hidden, seed=41)
    up = random_matrix(Q4_K, experts * mid, hidden, seed=42)
    down = random_matrix(Q4_K, experts * hidden, mid, seed=43)
    x = np.random.default_rng(44).normal(0, 1, (tokens, hidden)).astype(np.float32)
    x[5] *= 1e6
    x[9] *= 1e-6
    x = x.ravel()
    seed_out = np.random.default_rng(45).normal(0, 1, (tokens, hidden)).astype(np.float32)
    seed_out[9] = 0.0  # so row 9's check sees its 1e-6-scaled expert sum
    pt = list(range(40)) + [40, 41, 42, 5, 9, 0]
    pe = [3] * 40 + [7, 7, 11, 0, 0, 11]
    pw = np.random.default_rng(46).uniform(0.1, 1.0, len(pt)).astype(np.float32)
    perm = np.random.default_rng(47).permutation(len(pt))
    pt, pe, pw = np.array(pt, np.int32)[perm], np.array(pe, np.int32)[perm], pw[perm]
    G = gpu_ctx.upload(Q4_K, gate, (hidden, mid, experts))
    U = gpu_ctx.upload(Q4_K, up, (hidden, mid, experts))
    D = gpu_ctx.upload(Q4_K, down, (mid, hidden, experts))
    got = hyq.moe_experts(G, U, D, x, tokens, pt, pe, pw, seed_out).reshape(tokens, hidden)
    ref, mag = chain_f64(oracle, Q4_K, Q4_K, gate, up, down, hidden, mid, x, pt, pe, pw,
                         seed_out, range(tokens))
    for t in range(tokens):
        check_moe(got[t:t + 1], ref[t][None], mag[t][None], f"few-token row {t}")
    assert np.array_equal(got[43], seed_out[43])  # token 43 is routed nowhere


def test_moe_q4k_few_token_chunks_large_plan(gpu_ctx, hyq, oracle):
    """The Q4_K register kernels after a plan of more than 1024 pairs (the
    plan kernels that do not form the token operands in their launch, so
    separate launches do): 1600 pairs over 160 experts, 10 per expert on
    average, hidden = mid = 256 (one superblock per row); 12 seeded tokens
    checked against the f64 chain."""
    hidden, mid, experts, tokens, used = 256, 256, 160, 200, 8
    _print("moe few-token chunks, 1600 pairs")
    gate = random_matrix(Q4_K, experts * mid, hidden, seed=61)
    up = random_matrix(Q4_K, experts * mid, hidden, seed=62)
    down = random_matrix(Q4_K, experts * hidden, mid, seed=63)
    x = np.random.default_rng(64).normal(0, 1, tokens * hidden).astype(np.float32)
    seed_out = np.random.default_rng(65).normal(0, 1, (tokens, hidden)).astype(np.float32)
    pt, pe, pw = routed_pairs(tokens, experts, used, seed=66)
    G = gpu_ctx.upload(Q4_K, gate, (hidden, mid, experts))
    U = gpu_ctx.upload(Q4_K, up, (hidden, mid, experts))
    D = gpu_ctx.upload(Q4_K, down, (mid, hidden, experts))
    got = hyq.moe_experts(G, U, D, x, tokens, pt, pe, pw, seed_out).reshape(tokens, hidden)
    assert np.all(np.isfinite(got))
    pick = sorted(np.random.default_rng(67).choice(tokens, 12, replace=False).tolist())
    ref, mag = chain_f64(oracle, Q4_K, Q4_K, gate, up, down, hidden, mid, x, pt, pe, pw,
                         seed_out, pick)
    check_moe(got[pick], np.stack([ref[t] for t in pick]), np.stack([mag[t] for t in pick]),
              "few-token chunks, 1600 pairs")


def test_moe_30b_a3b_shape_sampled_tokens(gpu_ctx, hyq, oracle):
    """64 tokens, top-8 of 64 experts (softmax routing), hidden 2048, mid 1536,
    Q4_K experts; every token's output is produced, 6 seeded tokens are
    checked against the f64 chain."""
    hidden, mid, experts, tokens, used = 2048, 1536, 64, 64, 8
    _print("moe 30B-A3B shape")
    gate = random_matrix(Q4_K, experts * mid, hidden, seed=21)
    up = random_matrix(Q4_K, experts * mid, hidden, seed=22)
    down = random_matrix(Q4_K, experts * hidden, mid, seed=23)
    x = np.random.default_rng(24).normal(0, 1, tokens * hidden).astype(np.float32)
    seed_out = np.random.default_rng(25).normal(0, 1, (tokens, hidden)).astype(np.float32)
    pt, pe, pw = routed_pairs(tokens, experts, used, seed=26)
    G = gpu_ctx.upload(Q4_K, gate, (hidden, mid, experts))
    U = gpu_ctx.upload(Q4_K, up, (hidden, mid, experts))
    D = gpu_ctx.upload(Q4_K, down, (mid, hidden, experts))
    got = hyq.moe_experts(G, U, D, x, tokens, pt, pe, pw, seed_out).reshape(tokens, hidden)
    assert np.all(np.isfinite(got))
    pick = sorted(np.random.default_rng(27).choice(tokens, 6, replace=False).tolist())
    ref, mag = chain_f64(oracle, Q4_K, Q4_K, gate, up, down, hidden, mid, x, pt, pe, pw,
                         seed_out, pick)
    check_moe(got[pick], np.stack([ref[t] for t in pick]), np.stack([mag[t] for t in pick]),
              "30B-A3B")


@pytest.mark.parametrize("hidden,mid", [(2048, 1024), (4096, 512), (2048, 768), (1024, 1536)])
def test_moe_row_group_streams(gpu_ctx, hyq, oracle, hidden, mid):
    """Workgroups that stream several row groups against one activation copy
    (gate/up: 4 or 6 groups of 64 rows; down: groups of 128 rows), with K
    slices of 2, 4, 6 and 8 superblocks (the register ring in whole rounds
    per group or per pair of groups) and of 3 (one group): every token
    checked against the f64 chain."""
    experts, tokens, used = 8, 24, 3
    _print(f"moe row groups hidden {hidden} mid {mid}")
    gate = random_matrix(Q4_K, experts * mid, hidden, seed=51)
    up = random_matrix(Q4_K, experts * mid, hidden, seed=52)
    down = random_matrix(Q4_K, experts * hidden, mid, seed=53)
    x = np.random.default_rng(54).normal(0, 1, tokens * hidden).astype(np.float32)
    seed_out = np.random.default_rng(55).normal(0, 1, (tokens, hidden)).astype(np.float32)
    pt, pe, pw = routed_pairs(tokens, experts, used, seed=56)
    G = gpu_ctx.upload(Q4_K, gate, (hidden, mid, experts))
    U = gpu_ctx.upload(Q4_K, up, (hidden, mid, experts))
    D = gpu_ctx.upload(Q4_K, down, (mid, hidden, experts))
    got = hyq.moe_experts(G, U, D, x, tokens, pt, pe, pw, seed_out).reshape(tokens, hidden)
    ref, mag = chain_f64(oracle, Q4_K, Q4_K, gate, up, down, hidden, mid, x, pt, pe, pw,
                         seed_out, range(tokens))
    check_moe(got, np.stack([ref[t] for t in range(tokens)]),
              np.stack([mag[t] for t in range(tokens)]), f"row groups {hidden}x{mid}")


def test_moe_device_entry_point_and_rerun(gpu_ctx, hyq):
    """hyq_moe_experts_d on device buffers equals the host entry point, twice
    in a row on the same scratch (the second with fewer pairs)."""
    hidden, mid, experts, tokens = 256, 256, 4, 10
    gate = random_matrix(Q4_K, experts * mid, hidden, seed=31)
    up = random_matrix(Q4_K, experts * mid, hidden, seed=32)
    down = random_matrix(Q4_K, experts * hidden, mid, seed=33)
    x = np.random.default_rng(34).normal(0, 1, tokens * hidden).astype(np.float32)
    G = gpu_ctx.upload(Q4_K, gate, (hidden, mid, experts))
    U = gpu_ctx.upload(Q4_K, up, (hidden, mid, experts))
    D = gpu_ctx.upload(Q4_K, down, (mid, hidden, experts))
    L = hyq.lib()
    nbytes = L.hyq_moe_scratch_bytes(tokens, 20, experts, hidden, mid)
    scratch = gpu_ctx.empty(nbytes, np.uint8)
    xd = gpu_ctx.array(x)
    for npairs in (20, 7):
        pt, pe, pw = routed_pairs(tokens, experts, 2, seed=npairs)
        pt, pe, pw = pt[:npairs], pe[:npairs], pw[:npairs]
        host = hyq.moe_experts(G, U, D, x, tokens, pt, pe, pw,
                               np.zeros(tokens * hidden, np.float32))
        od = gpu_ctx.array(np.zeros(tokens * hidden, np.float32))
        ptd, ped, pwd = gpu_ctx.array(pt), gpu_ctx.array(pe), gpu_ctx.array(pw)
        hyq.check(L.hyq_moe_experts_d(gpu_ctx.handle, G.handle, U.handle, D.handle, xd.ptr,
                                      tokens, ptd.ptr, ped.ptr, pwd.ptr, npairs, scratch.ptr,
                                      nbytes, od.ptr))
        assert np.array_equal(od.numpy(), host)


@pytest.mark.parametrize("tokens,used", [(64, 8), (100, 8), (1, 8), (16, 0)])
def test_moe_shared_experts_matches_two_calls(gpu_ctx, hyq, oracle, tokens, used):
    """hyq_moe_shared_experts_d at the 30B-A3B layer shape (Q8_0 shared
    projection [2048x2048], top-`used` of 64 Q4_K experts): at 64 and 100
    tokens the shared product's tiles run inside the expert launches (one and
    two 64-token chunk groups), at one token or with no pairs the two calls
    run. Five calls in a row, the output refilled with NaN before each (a
    seed the shared tiles failed to write would keep them), each equal bit for
    bit to hyq_matmul_d followed by hyq_moe_experts_d; three tokens against
    the f64 chain seeded with the oracle's shared product. Token rows 5 and 9
    are scaled by 1e6 and 1e-6."""
    hidden, mid, experts = 2048, 1536, 64
    _print("moe shared + experts", tokens, used)
    gate = random_matrix(Q4_K, experts * mid, hidden, seed=41)
    up = random_matrix(Q4_K, experts * mid, hidden, seed=42)
    down = random_matrix(Q4_K, experts * hidden, mid, seed=43)
    shared = random_matrix(Q8_0, hidden, hidden, seed=44)
    x = np.random.default_rng(45).normal(0, 1, (tokens, hidden)).astype(np.float32)
    if tokens > 10:  # the f16 row scales of both products' operands
        x[5] *= 1e6
        x[9] *= 1e-6
    x = x.ravel()
    if used:
        pt, pe, pw = routed_pairs(tokens, experts, used, seed=46)
    else:
        pt = pe = np.zeros(0, np.int32)
        pw = np.zeros(0, np.float32)
    G = gpu_ctx.upload(Q4_K, gate, (hidden, mid, experts))
    U = gpu_ctx.upload(Q4_K, up, (hidden, mid, experts))
    D = gpu_ctx.upload(Q4_K, down, (mid, hidden, experts))
    S = gpu_ctx.upload(Q8_0, shared, (hidden, hidden))
    L = hyq.lib()
    n = len(pt)
    nbytes = L.hyq_moe_scratch_bytes(tokens, max(n, 1), experts, hidden, mid)
    scratch = gpu_ctx.empty(nbytes, np.uint8)
    xd = gpu_ctx.array(x)
    ptd, ped, pwd = (gpu_ctx.array(a if n else np.zeros(1, a.dtype)) for a in (pt, pe, pw))
    seq = gpu_ctx.empty(tokens * hidden, np.float32)
    hyq.check(L.hyq_matmul_d(gpu_ctx.handle, S.handle, xd.ptr, tokens, seq.ptr))
    hyq.check(L.hyq_moe_experts_d(gpu_ctx.handle, G.handle, U.handle, D.handle, xd.ptr, tokens,
                                  ptd.ptr, ped.ptr, pwd.ptr, n, scratch.ptr, nbytes, seq.ptr))
    want = seq.numpy()
    nan = np.full(tokens * hidden, np.nan, np.float32)
    od = gpu_ctx.array(nan)
    for i in range(5):
        od.copy_from(nan)
        hyq.check(L.hyq_moe_shared_experts_d(gpu_ctx.handle, S.handle, G.handle, U.handle,
                                             D.handle, xd.ptr, tokens, ptd.ptr, ped.ptr, pwd.ptr,
                                             n, scratch.ptr, nbytes, od.ptr))
        got = od.numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (tokens, used, i)
    pick = sorted(np.random.default_rng(47).choice(tokens, min(3, tokens),
                                                   replace=False).tolist())
    seed = np.zeros((tokens, hidden), np.float64)
    smag = np.zeros((tokens, hidden))
    for t in pick:
        y, m = oracle.matmul_f64(Q8_0, shared, hidden, hidden, x[t * hidden:(t + 1) * hidden], 1)
        seed[t], smag[t] = y[0], m[0]
    ref, mag = chain_f64(oracle, Q4_K, Q4_K, gate, up, down, hidden, mid, x, pt, pe, pw, seed,
                         pick)
    got = want.reshape(tokens, hidden)
    check_moe(got[pick], np.stack([ref[t] for t in pick]),
              np.stack([mag[t] + smag[t] for t in pick]), f"shared + experts {tokens}")
    for w in (G, U, D, S):
        w.release()


def test_moe_errors(gpu_ctx, hyq):
    hidden, mid, experts = 256, 512, 4
    G = gpu_ctx.upload(Q4_K, random_matrix(Q4_K, experts * mid, hidden, seed=1),
                       (hidden, mid, experts))
    D = gpu_ctx.upload(Q4_K, random_matrix(Q4_K, experts * hidden, mid, seed=2),
                       (mid, hidden, experts))
    x = np.zeros(2 * hidden, np.float32)
    out = np.zeros(2 * hidden, np.float32)
    with pytest.raises(ValueError):  # expert out of range
        hyq.moe_experts(G, G, D, x, 2, [0], [4], [1.0], out)
    with pytest.raises(ValueError):  # token out of range
        hyq.moe_experts(G, G, D, x, 2, [2], [0], [1.0], out)
    with pytest.raises(ValueError):  # down given where gate is expected
        hyq.moe_experts(D, G, D, x, 2, [0], [0], [1.0], out)
    assert np.array_equal(hyq.moe_experts(G, G, D, x, 2, [], [], [], out), out)
