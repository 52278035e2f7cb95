"""A small GGUF v3 writer for tests: builds files whose every field the test
chooses (including malformed ones), and a hunyuan-dense model file from a
synthetic model dict (tests/synth.py:make_dense_model)."""
from __future__ import annotations

import struct

import numpy as np

# metadata value types (GGUF v3)
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
        U64: "<Q", I64: "<q", F64: "<d"}


def string(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def value(kind: int, v) -> bytes:
    if kind in _FMT:
        return struct.pack(_FMT[kind], v)
    if kind == BOOL:
        return struct.pack("<B", int(v))
    if kind == STR:
        return string(v)
    if kind == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(value(et, x) for x in items)
    raise ValueError(kind)


def build(meta: list, tensors: list, alignment: int = 32, version: int = 3) -> bytes:
    """meta: [(key, kind, value)]; tensors: [(name, dims, type_id, data bytes)] laid out
    in order at aligned offsets (or (name, dims, type_id, data, offset) to force one)."""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta)))
    for key, kind, v in meta:
        out += string(key) + struct.pack("<I", kind) + value(kind, v)
    offsets, off, end = [], 0, 0
    for t in tensors:
        o = t[4] if len(t) == 5 else off
        offsets.append(o)
        end = max(end, o + len(t[3]))
        off = (end + alignment - 1) // alignment * alignment
    for t, o in zip(tensors, offsets):
        name, dims, type_id = t[0], t[1], t[2]
        out += string(name) + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", type_id, o)
    out += bytes(-len(out) % alignment)
    data = bytearray(end)  # no padding after the last tensor
    for t, o in zip(tensors, offsets):
        data[o:o + len(t[3])] = t[3]
    return bytes(out + data)


def dense_model_file(model: dict, linear_id: int, embed_id: int = 14, file_type: int | None = None,
                     context_length: int = 4096) -> bytes:
    """A hunyuan-dense GGUF of a synthetic model: linears stored with type id
    `linear_id` (40 = Q2_0C under the tencent-q2-0c profile, 42 = STQ1_0 under
    tencent-stq1), Q6_K (14) embedding and output, F32 (0) norm vectors."""
    c = model["cfg"]
    a = "hunyuan-dense"
    meta = [("general.architecture", STR, a)]
    if file_type is not None:
        meta.append(("general.file_type", U32, file_type))
    meta += [(f"{a}.block_count", U32, c["layers"]), (f"{a}.embedding_length", U32, c["hidden"]),
             (f"{a}.attention.head_count", U32, c["heads"]),
             (f"{a}.attention.head_count_kv", U32, c["kv_heads"]),
             (f"{a}.attention.key_length", U32, c["head_dim"]),
             (f"{a}.attention.value_length", U32, c["head_dim"]),
             (f"{a}.context_length", U32, context_length),
             (f"{a}.rope.freq_base", F32, c["rope_base"]),
             (f"{a}.attention.layer_norm_rms_epsilon", F32, c["rms_eps"]),
             (f"{a}.feed_forward_length", U32, c["ffn"]),
             ("tokenizer.ggml.model", STR, "gpt2"),
             ("tokenizer.ggml.tokens", ARR, (STR, [f"t{i}" for i in range(c["vocab"])]))]
    H, F, D = c["hidden"], c["ffn"], c["head_dim"]
    QL, KV = c["heads"] * D, c["kv_heads"] * D
    f32 = lambda v: np.ascontiguousarray(v, np.float32).tobytes()
    tensors = [("token_embd.weight", [H, c["vocab"]], embed_id, model["embed"].tobytes()),
               ("output_norm.weight", [H], 0, f32(model["output_norm"]))]
    if "output" in model:
        tensors.append(("output.weight", [H, c["vocab"]], embed_id, model["output"].tobytes()))
    for i, L in enumerate(model["layers"]):
        p = f"blk.{i}."
        tensors += [(p + "attn_norm.weight", [H], 0, f32(L["attn_norm"])),
                    (p + "ffn_norm.weight", [H], 0, f32(L["ffn_norm"])),
                    (p + "attn_q.weight", [H, QL], linear_id, L["q"].tobytes()),
                    (p + "attn_k.weight", [H, KV], linear_id, L["k"].tobytes()),
                    (p + "attn_v.weight", [H, KV], linear_id, L["v"].tobytes()),
                    (p + "attn_output.weight", [QL, H], linear_id, L["o"].tobytes()),
                    (p + "attn_q_norm.weight", [D], 0, f32(L["q_norm"])),
                    (p + "attn_k_norm.weight", [D], 0, f32(L["k_norm"])),
                    (p + "ffn_gate.weight", [H, F], linear_id, L["gate"].tobytes()),
                    (p + "ffn_up.weight", [H, F], linear_id, L["up"].tobytes()),
                    (p + "ffn_down.weight", [F, H], linear_id, L["down"].tobytes())]
    return build(meta, tensors)


def hyv3_model_file(model: dict, linear_id: int = 12, embed_id: int = 14, expert_id: int = 12,
                    shared_id: int = 8, context_length: int = 4096,
                    gating: int = 2, drop: str | None = None,
                    router_f16: bool = False) -> bytes:
    """A hy_v3 GGUF of a synthetic model (tests/synth.py:make_hyv3_model):
    layer 0 with a dense FFN, later layers with an F32 router, the
    exp_probs_b bias, expert stacks and a shared expert; `drop` leaves out
    one tensor by name; router_f16 stores the routers as F16 (type 1)."""
    c = model["cfg"]
    a = "hy_v3"
    moe = next(L["moe"] for L in model["layers"] if "moe" in L)
    meta = [("general.architecture", STR, a),
            (f"{a}.block_count", U32, c["layers"]), (f"{a}.embedding_length", U32, c["hidden"]),
            (f"{a}.attention.head_count", U32, c["heads"]),
            (f"{a}.attention.head_count_kv", U32, c["kv_heads"]),
            (f"{a}.attention.key_length", U32, c["head_dim"]),
            (f"{a}.attention.value_length", U32, c["head_dim"]),
            (f"{a}.context_length", U32, context_length),
            (f"{a}.rope.freq_base", F32, c["rope_base"]),
            (f"{a}.attention.layer_norm_rms_epsilon", F32, c["rms_eps"]),
            (f"{a}.feed_forward_length", U32, c["ffn"]),
            (f"{a}.expert_count", U32, moe["experts"]),
            (f"{a}.expert_used_count", U32, moe["used"]),
            (f"{a}.expert_feed_forward_length", U32, moe["mid"]),
            (f"{a}.expert_shared_feed_forward_length", U32, moe["shared_mid"]),
            (f"{a}.expert_gating_func", U32, gating),
            (f"{a}.expert_weights_scale", F32, moe["scale"]),
            (f"{a}.expert_weights_norm", BOOL, bool(moe["normalize"])),
            ("tokenizer.ggml.model", STR, "gpt2"),
            ("tokenizer.ggml.tokens", ARR, (STR, [f"t{i}" for i in range(c["vocab"])]))]
    H, F, D = c["hidden"], c["ffn"], c["head_dim"]
    QL, KV = c["heads"] * D, c["kv_heads"] * D
    f32 = lambda v: np.ascontiguousarray(v, np.float32).tobytes()
    tensors = [("token_embd.weight", [H, c["vocab"]], embed_id, model["embed"].tobytes()),
               ("output_norm.weight", [H], 0, f32(model["output_norm"])),
               ("output.weight", [H, c["vocab"]], embed_id, model["output"].tobytes())]
    for i, L in enumerate(model["layers"]):
        p = f"blk.{i}."
        tensors += [(p + "attn_norm.weight", [H], 0, f32(L["attn_norm"])),
                    (p + "ffn_norm.weight", [H], 0, f32(L["ffn_norm"])),
                    (p + "attn_q.weight", [H, QL], linear_id, L["q"].tobytes()),
                    (p + "attn_k.weight", [H, KV], linear_id, L["k"].tobytes()),
                    (p + "attn_v.weight", [H, KV], linear_id, L["v"].tobytes()),
                    (p + "attn_output.weight", [QL, H], linear_id, L["o"].tobytes()),
                    (p + "attn_q_norm.weight", [D], 0, f32(L["q_norm"])),
                    (p + "attn_k_norm.weight", [D], 0, f32(L["k_norm"]))]
        if "moe" not in L:
            tensors += [(p + "ffn_gate.weight", [H, F], linear_id, L["gate"].tobytes()),
                        (p + "ffn_up.weight", [H, F], linear_id, L["up"].tobytes()),
                        (p + "ffn_down.weight", [F, H], linear_id, L["down"].tobytes())]
            continue
        e = L["moe"]
        E, M, S = e["experts"], e["mid"], e["shared_mid"]
        router = (("ffn_gate_inp.weight", [H, E], 1, e["router"].astype(np.float16).tobytes())
                  if router_f16 else ("ffn_gate_inp.weight", [H, E], 0, f32(e["router"])))
        tensors += [(p + router[0], router[1], router[2], router[3]),
                    (p + "exp_probs_b", [E], 0, f32(e["bias"])),
                    (p + "ffn_gate_exps.weight", [H, M, E], expert_id, e["gate"].tobytes()),
                    (p + "ffn_up_exps.weight", [H, M, E], expert_id, e["up"].tobytes()),
                    (p + "ffn_down_exps.weight", [M, H, E], expert_id, e["down"].tobytes()),
                    (p + "ffn_gate_shexp.weight", [H, S], shared_id, e["sgate"].tobytes()),
                    (p + "ffn_up_shexp.weight", [H, S], shared_id, e["sup"].tobytes()),
                    (p + "ffn_down_shexp.weight", [S, H], shared_id, e["sdown"].tobytes())]
    if drop is not None:
        tensors = [t for t in tensors if t[0] != drop]
    return build(meta, tensors)
