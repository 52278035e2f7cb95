"""Seeded synthetic quantized weights for tests and benchmarks.

Block recipes follow the workload descriptions of the quantized matmul path:
  fp16 scales      |N(0, 0.02)| (Q4_K d and dmin, Q2_0C d, STQ d, Q6_K d,
                   Q8_0 d), always finite and nonzero unless overridden;
  Q4_K             6-bit sub-scales and mins uniform 0..63 (packed as the
                   decoder reads them, src/quant.rs:2441-2451), nibbles uniform;
  Q2_0C            uniform code bytes;
  STQ1_0           uniform nibble and sign bytes (exactly 25% zero digits,
                   fixed by the codebook);
  Q6_K             uniform ql/qh bytes, uniform int8 sub-scales;
  Q8_0             uniform int8 quants.
"""
from __future__ import annotations

import numpy as np

F32, F16, Q8_0, Q4_K, Q6_K, Q2_0C, STQ1_0 = 0, 1, 8, 12, 14, 40, 42
BLOCK_LEN = {F32: 1, F16: 1, Q8_0: 32, Q4_K: 256, Q6_K: 256, Q2_0C: 512, STQ1_0: 256}
BLOCK_BYTES = {F32: 4, F16: 2, Q8_0: 34, Q4_K: 144, Q6_K: 210, Q2_0C: 130, STQ1_0: 42}
NAMES = {F32: "F32", F16: "F16", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K",
         Q2_0C: "Q2_0C", STQ1_0: "STQ1_0"}
QUANT = (Q2_0C, STQ1_0, Q4_K, Q6_K, Q8_0)


def row_bytes(dtype: int, cols: int) -> int:
    return cols // BLOCK_LEN[dtype] * BLOCK_BYTES[dtype]


def _f16_scales(rng: np.random.Generator, n: int, sigma: float = 0.02) -> np.ndarray:
    v = np.abs(rng.normal(0.0, sigma, n)).astype(np.float16)
    v[v == 0] = np.float16(sigma)
    return v


def random_blocks(dtype: int, nblocks: int, seed: int = 0) -> np.ndarray:
    """nblocks packed blocks of dtype as a flat uint8 array."""
    rng = np.random.default_rng(seed)
    bb = BLOCK_BYTES[dtype]
    b = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    if dtype == Q2_0C:
        b[:, 0:2] = _f16_scales(rng, nblocks).view(np.uint8).reshape(nblocks, 2)
    elif dtype == STQ1_0:
        b[:, 40:42] = _f16_scales(rng, nblocks).view(np.uint8).reshape(nblocks, 2)
    elif dtype == Q8_0:
        b[:, 0:2] = _f16_scales(rng, nblocks).view(np.uint8).reshape(nblocks, 2)
    elif dtype == Q6_K:
        b[:, 208:210] = _f16_scales(rng, nblocks).view(np.uint8).reshape(nblocks, 2)
    elif dtype == Q4_K:
        b[:, 0:2] = _f16_scales(rng, nblocks).view(np.uint8).reshape(nblocks, 2)
        b[:, 2:4] = _f16_scales(rng, nblocks).view(np.uint8).reshape(nblocks, 2)
        s = rng.integers(0, 64, size=(nblocks, 8), dtype=np.uint8)
        m = rng.integers(0, 64, size=(nblocks, 8), dtype=np.uint8)
        b[:, 4:16] = pack_q4k_scales(s, m)
    elif dtype == F32:
        b = rng.normal(0, 1, nblocks).astype(np.float32).view(np.uint8).reshape(nblocks, 4)
    elif dtype == F16:
        b = rng.normal(0, 1, nblocks).astype(np.float16).view(np.uint8).reshape(nblocks, 2)
    return np.ascontiguousarray(b).reshape(-1)


def pack_q4k_scales(s: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Inverse of the 6-bit unpacking of src/quant.rs:2441-2451 (per row of 8)."""
    n = s.shape[0]
    out = np.zeros((n, 12), dtype=np.uint8)
    for j in range(4):
        out[:, j] = (s[:, j] & 63) | ((s[:, j + 4] >> 4) << 6)
        out[:, j + 4] = (m[:, j] & 63) | ((m[:, j + 4] >> 4) << 6)
        out[:, j + 8] = (s[:, j + 4] & 15) | ((m[:, j + 4] & 15) << 4)
    return out


def random_matrix(dtype: int, rows: int, cols: int, seed: int = 0) -> np.ndarray:
    nb = rows * cols // BLOCK_LEN[dtype]
    return random_blocks(dtype, nb, seed)


def set_block_scale(dtype: int, blocks: np.ndarray, value: float, dmin: float | None = None):
    """Overwrite every block's fp16 scale (and Q4_K dmin) in place."""
    bb = BLOCK_BYTES[dtype]
    b = blocks.reshape(-1, bb)
    h = np.array([value], dtype=np.float16).view(np.uint8)
    off = {Q2_0C: 0, STQ1_0: 40, Q8_0: 0, Q6_K: 208, Q4_K: 0}[dtype]
    b[:, off:off + 2] = h
    if dtype == Q4_K and dmin is not None:
        b[:, 2:4] = np.array([dmin], dtype=np.float16).view(np.uint8)
    return blocks


# ---------------------------------------------------------------------------
# Synthetic dense model (random-init weights of the hunyuan-dense shape)
# ---------------------------------------------------------------------------
DENSE_1P8B = dict(layers=32, hidden=2048, heads=16, kv_heads=4, head_dim=128, ffn=6144,
                  vocab=120818, rope_base=11158840.0, rms_eps=1e-5)


def make_dense_model(cfg: dict, linear: int = Q2_0C, embed: int = Q6_K, seed: int = 0,
                     down: int | None = None) -> dict:
    """Packed GGUF bytes for every matrix plus f32 norms ~ N(1, 0.02).
    The output matrix is tied to the embedding (src/model.rs:194-202).
    `down` gives ffn_down its own format (Q6_K in the Q4_K_M mix)."""
    down = linear if down is None else down
    rng = np.random.default_rng(seed)
    H, F, D = cfg["hidden"], cfg["ffn"], cfg["head_dim"]
    QL, KV = cfg["heads"] * D, cfg["kv_heads"] * D
    layers = []
    for l in range(cfg["layers"]):
        s = seed * 1000 + l * 10
        layers.append(dict(
            q=random_matrix(linear, QL, H, s + 1), k=random_matrix(linear, KV, H, s + 2),
            v=random_matrix(linear, KV, H, s + 3), o=random_matrix(linear, H, QL, s + 4),
            gate=random_matrix(linear, F, H, s + 5), up=random_matrix(linear, F, H, s + 6),
            down=random_matrix(down, H, F, s + 7),
            attn_norm=rng.normal(1, 0.02, H).astype(np.float32),
            ffn_norm=rng.normal(1, 0.02, H).astype(np.float32),
            q_norm=rng.normal(1, 0.02, D).astype(np.float32),
            k_norm=rng.normal(1, 0.02, D).astype(np.float32)))
    return dict(cfg=dict(cfg), linear=linear, down_dtype=down, embed_dtype=embed, layers=layers,
                embed=random_matrix(embed, cfg["vocab"], H, seed * 1000 + 999),
                output_norm=rng.normal(1, 0.02, H).astype(np.float32))


def make_hyv3_model(cfg: dict, moe: dict, linear: int = Q4_K, expert: int = Q4_K,
                    shared: int = Q8_0, embed: int = Q6_K, seed: int = 0) -> dict:
    """A synthetic hy_v3 model (src/model.rs:136-262): layer 0 keeps a dense
    FFN of width cfg["ffn"], every later layer an MoE FFN of `moe`'s shape
    (experts, used, mid, shared_mid, normalize, scale) with an F32 router
    ~ N(0, 1/sqrt(hidden)) (router logits ~ N(0, 1)), a selection bias
    ~ N(0, 0.1), Q4_K expert stacks and a Q8_0 shared expert; a separate
    output matrix (HyV3 requires one, src/model.rs:194-201)."""
    model = make_dense_model(cfg, linear=linear, embed=embed, seed=seed)
    model["arch"] = 1
    H, V = cfg["hidden"], cfg["vocab"]
    E, mid, smid = moe["experts"], moe["mid"], moe["shared_mid"]
    model["output"] = random_matrix(embed, V, H, seed * 1000 + 998)
    rng = np.random.default_rng(seed + 777)
    for l in range(1, cfg["layers"]):
        L = model["layers"][l]
        for k in ("gate", "up", "down"):
            del L[k]
        s = seed * 1000 + l * 10 + 500
        L["moe"] = dict(
            moe, dtype_gate=expert, dtype_down=expert, dtype_shared=shared,
            dtype_shared_down=shared,
            router=(rng.normal(0, 1, (E, H)) / np.sqrt(H)).astype(np.float32),
            bias=rng.normal(0, 0.1, E).astype(np.float32),
            gate=random_matrix(expert, E * mid, H, s + 1),
            up=random_matrix(expert, E * mid, H, s + 2),
            down=random_matrix(expert, E * H, mid, s + 3),
            sgate=random_matrix(shared, smid, H, s + 4),
            sup=random_matrix(shared, smid, H, s + 5),
            sdown=random_matrix(shared, H, smid, s + 6))
    return model


def make_kv_cache(cfg: dict, context: int, prefilled: int, seed: int = 0):
    """f32 K/V caches [layers][context][kv_heads*head_dim], N(0,1) up to prefilled."""
    rng = np.random.default_rng(seed + 12345)
    kvw = cfg["kv_heads"] * cfg["head_dim"]
    k = np.zeros((cfg["layers"], context, kvw), np.float32)
    v = np.zeros((cfg["layers"], context, kvw), np.float32)
    k[:, :prefilled] = rng.standard_normal((cfg["layers"], prefilled, kvw), np.float32)
    v[:, :prefilled] = rng.standard_normal((cfg["layers"], prefilled, kvw), np.float32)
    return k, v


def dense_weight_bytes(model: dict) -> int:
    """Packed weight bytes one decode step streams (tied embedding read once)."""
    total = sum(a.size for L in model["layers"] for n, a in L.items()
                if a.dtype == np.uint8)
    return total + model["embed"].size


def load_dense(hyq, ctx, model: dict, context: int):
    """Upload a synthetic model into a hyq DenseDecoder (weights kept alive on it)."""
    c = model["cfg"]
    cfg = hyq.DenseConfig(c["layers"], c["hidden"], c["heads"], c["kv_heads"], c["head_dim"],
                          c["ffn"], c["vocab"], c["rope_base"], c["rms_eps"])
    dec = hyq.DenseDecoder(ctx, cfg, context)
    H, F, D = c["hidden"], c["ffn"], c["head_dim"]
    QL, KV = c["heads"] * D, c["kv_heads"] * D
    lin = model["linear"]
    for l, L in enumerate(model["layers"]):
        W = dict(q=ctx.upload(lin, L["q"], (H, QL)), k=ctx.upload(lin, L["k"], (H, KV)),
                 v=ctx.upload(lin, L["v"], (H, KV)), o=ctx.upload(lin, L["o"], (QL, H)),
                 gate=ctx.upload(lin, L["gate"], (H, F)), up=ctx.upload(lin, L["up"], (H, F)),
                 down=ctx.upload(model.get("down_dtype", lin), L["down"], (F, H)))
        dec.set_layer(l, W["q"], W["k"], W["v"], W["o"], W["gate"], W["up"], W["down"],
                      L["attn_norm"], L["ffn_norm"], L["q_norm"], L["k_norm"])
    E = ctx.upload(model["embed_dtype"], model["embed"], (H, c["vocab"]))
    O = E
    if "output" in model:
        O = ctx.upload(model["embed_dtype"], model["output"], (H, c["vocab"]))
    dec.set_output(E, O, model["output_norm"])
    return dec


def upload_moe(hyq, ctx, moe: dict, hidden: int):
    """A synthetic MoE FFN (make_hyv3_model's layer["moe"]) as a hyq.MoeFfn."""
    E, mid, smid = moe["experts"], moe["mid"], moe["shared_mid"]
    cfg = hyq.MoeConfig(E, moe["used"], mid, smid, int(moe["normalize"]), moe["scale"])
    router = ctx.upload(F32, moe["router"].view(np.uint8).reshape(-1), (hidden, E))
    g = ctx.upload(moe["dtype_gate"], moe["gate"], (hidden, mid, E))
    u = ctx.upload(moe["dtype_gate"], moe["up"], (hidden, mid, E))
    d = ctx.upload(moe["dtype_down"], moe["down"], (mid, hidden, E))
    sg = ctx.upload(moe["dtype_shared"], moe["sgate"], (hidden, smid))
    su = ctx.upload(moe["dtype_shared"], moe["sup"], (hidden, smid))
    sd = ctx.upload(moe["dtype_shared_down"], moe["sdown"], (smid, hidden))
    return hyq.MoeFfn(ctx, cfg, router, moe["bias"], g, u, d, sg, su, sd)


def load_hyv3(hyq, ctx, model: dict, context: int):
    """Upload a synthetic hy_v3 model (make_hyv3_model) into a decoder."""
    c = model["cfg"]
    cfg = hyq.DenseConfig(c["layers"], c["hidden"], c["heads"], c["kv_heads"], c["head_dim"],
                          c["ffn"], c["vocab"], c["rope_base"], c["rms_eps"])
    dec = hyq.DenseDecoder(ctx, cfg, context)
    dec.set_architecture(hyq.ARCH_HYV3)
    H, F, D = c["hidden"], c["ffn"], c["head_dim"]
    QL, KV = c["heads"] * D, c["kv_heads"] * D
    lin = model["linear"]
    for l, L in enumerate(model["layers"]):
        W = dict(q=ctx.upload(lin, L["q"], (H, QL)), k=ctx.upload(lin, L["k"], (H, KV)),
                 v=ctx.upload(lin, L["v"], (H, KV)), o=ctx.upload(lin, L["o"], (QL, H)))
        if "moe" in L:
            W.update(gate=None, up=None, down=None)
        else:
            W.update(gate=ctx.upload(lin, L["gate"], (H, F)), up=ctx.upload(lin, L["up"], (H, F)),
                     down=ctx.upload(model.get("down_dtype", lin), L["down"], (F, H)))
        dec.set_layer(l, W["q"], W["k"], W["v"], W["o"], W["gate"], W["up"], W["down"],
                      L["attn_norm"], L["ffn_norm"], L["q_norm"], L["k_norm"])
        if "moe" in L:
            dec.set_moe(l, upload_moe(hyq, ctx, L["moe"], H))
    E = ctx.upload(model["embed_dtype"], model["embed"], (H, c["vocab"]))
    O = ctx.upload(model["embed_dtype"], model["output"], (H, c["vocab"]))
    dec.set_output(E, O, model["output_norm"])
    return dec
