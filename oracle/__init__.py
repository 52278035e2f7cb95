"""ctypes binding of the CPU oracle (oracle/libhyq_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package. The C sources
restate the reference's algorithms; hyq_oracle.h lists what pins each one.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhyq_oracle.so")

F32, F16, Q8_0, Q4_K, Q6_K, Q2_0C, STQ1_0 = 0, 1, 8, 12, 14, 40, 42
NAMES = {"F32": F32, "F16": F16, "Q8_0": Q8_0, "Q4_K": Q4_K, "Q6_K": Q6_K,
         "Q2_0C": Q2_0C, "STQ1_0": STQ1_0}
BLOCK_LEN = {F32: 1, F16: 1, Q8_0: 32, Q4_K: 256, Q6_K: 256, Q2_0C: 512, STQ1_0: 256}
BLOCK_BYTES = {F32: 4, F16: 2, Q8_0: 34, Q4_K: 144, Q6_K: 210, Q2_0C: 130, STQ1_0: 42}


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = ctypes.c_void_p
SZ = ctypes.c_size_t
I = ctypes.c_int


def _declare(L: ctypes.CDLL) -> None:
    sig = {
        "hyqo_block_len": (ctypes.c_int, [ctypes.c_int]),
        "hyqo_block_bytes": (ctypes.c_int, [ctypes.c_int]),
        "hyqo_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "hyqo_decode": (ctypes.c_int, [ctypes.c_int, P, SZ, P, SZ]),
        "hyqo_q8_quantize": (None, [P, SZ, P, P]),
        "hyqo_q8_deinterleave_q2c": (None, [P, SZ, P]),
        "hyqo_row_isums": (ctypes.c_int, [ctypes.c_int, P, SZ, P, P]),
        "hyqo_isums_per_row": (ctypes.c_int, [ctypes.c_int, SZ]),
        "hyqo_gemv_q8_f64": (None, [ctypes.c_int, P, SZ, SZ, P, P, P, P]),
        "hyqo_gemv_q8_bruteforce": (None, [ctypes.c_int, P, SZ, SZ, P, P, P, P]),
        "hyqo_dot": (ctypes.c_float, [P, P, SZ]),
        "hyqo_dot_scalar": (ctypes.c_float, [P, P, SZ]),
        "hyqo_row_dot_f32": (ctypes.c_float, [ctypes.c_int, P, SZ, P]),
        "hyqo_matmul": (ctypes.c_int, [ctypes.c_int, P, SZ, SZ, P, SZ, P, ctypes.c_int]),
        "hyqo_gate_up_silu": (ctypes.c_int, [ctypes.c_int, P, P, SZ, SZ, P, P, ctypes.c_int]),
        "hyqo_matmul_f64": (None, [ctypes.c_int, P, SZ, SZ, P, SZ, P, P]),
        "hyqo_chunk_rows": (SZ, [SZ, ctypes.c_int]),
        "hyqo_route": (None, [P, P, SZ, SZ, ctypes.c_int, ctypes.c_float, P, P]),
        "hyqo_moe_experts": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, P, P, P, SZ, SZ, SZ,
                                            P, SZ, P, P, P, SZ, P, ctypes.c_int]),
        "hyqo_rms_norm_into": (None, [P, P, SZ, ctypes.c_float, P, I]),
        "hyqo_rms_norm_rows": (None, [P, P, SZ, SZ, ctypes.c_float, I]),
        "hyqo_rope_tables": (None, [SZ, ctypes.c_float, SZ, P, P]),
        "hyqo_rope": (None, [P, SZ, SZ, P, P]),
        "hyqo_attention": (None, [P, P, P, SZ, SZ, SZ, SZ, P]),
        "hyqo_decode_step": (ctypes.c_int, [P, P, P, SZ, SZ, ctypes.c_int, ctypes.c_int, P,
                                            ctypes.c_int]),
        "hyqo_prefill_chunk": (ctypes.c_int, [P, P, P, SZ, SZ, P, SZ, ctypes.c_int, P,
                                              ctypes.c_int]),
        "hyqo_layer_step": (ctypes.c_int, [P, ctypes.c_int, P, P, P, SZ, SZ, ctypes.c_int,
                                           ctypes.c_int]),
        "hyqo_prefill_layer": (ctypes.c_int, [P, ctypes.c_int, P, P, P, SZ, SZ, SZ,
                                              ctypes.c_int]),
        "hyqo_output_logits": (None, [P, P, ctypes.c_int, P, ctypes.c_int]),
        "hyqo_argmax": (ctypes.c_int, [P, SZ]),
        "hyqo_moe_forward": (None, [P, SZ, P, SZ, P, ctypes.c_int, ctypes.c_int]),
        "hyqo_moe_forward_tap": (None, [P, SZ, P, P, ctypes.c_int, P]),
        "hyqo_layer_step_tap": (ctypes.c_int, [P, ctypes.c_int, P, P, P, SZ, SZ, ctypes.c_int,
                                               P]),
        "hyqo_output_logits_tap": (None, [P, P, P, ctypes.c_int, P]),
        "hyqo_max_threads": (ctypes.c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def row_bytes(dtype: int, cols: int) -> int:
    return cols // BLOCK_LEN[dtype] * BLOCK_BYTES[dtype]


def decode(dtype: int, data: np.ndarray | bytes, n: int | None = None) -> np.ndarray:
    buf = np.frombuffer(bytes(data), dtype=np.uint8) if not isinstance(data, np.ndarray) else data
    buf = np.ascontiguousarray(buf, dtype=np.uint8)
    if n is None:
        n = buf.size // BLOCK_BYTES[dtype] * BLOCK_LEN[dtype]
    out = np.empty(n, dtype=np.float32)
    rc = lib().hyqo_decode(dtype, _p(buf), buf.size, _p(out), n)
    if rc != 0:
        raise ValueError(f"decode: invalid shape for dtype {dtype}")
    return out


def q8_quantize(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.size, dtype=np.int8)
    s = np.empty((x.size + 255) // 256, dtype=np.float32)
    lib().hyqo_q8_quantize(_p(x), x.size, _p(q), _p(s))
    return q, s


def q8_deinterleave_q2c(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int8)
    out = np.empty_like(q)
    lib().hyqo_q8_deinterleave_q2c(_p(q), q.size, _p(out))
    return out


def row_isums(dtype: int, row: np.ndarray, cols: int, q: np.ndarray) -> np.ndarray:
    per = lib().hyqo_isums_per_row(dtype, cols)
    out = np.empty(per, dtype=np.int32)
    row = np.ascontiguousarray(row, dtype=np.uint8)
    q = np.ascontiguousarray(q, dtype=np.int8)
    n = lib().hyqo_row_isums(dtype, _p(row), cols, _p(q), _p(out))
    assert n == per
    return out


def isums(dtype: int, w: np.ndarray, rows: int, cols: int, q: np.ndarray) -> np.ndarray:
    rb = row_bytes(dtype, cols)
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(rows, rb)
    return np.stack([row_isums(dtype, w[r], cols, q) for r in range(rows)])


def gemv_q8_f64(dtype: int, w: np.ndarray, rows: int, cols: int, q: np.ndarray,
                s: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    y = np.empty(rows, dtype=np.float64)
    mag = np.empty(rows, dtype=np.float64)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    lib().hyqo_gemv_q8_f64(dtype, _p(w), rows, cols, _p(q), _p(s), _p(y), _p(mag))
    return y, mag


def gemv_q8_bruteforce(dtype: int, w: np.ndarray, rows: int, cols: int, q: np.ndarray,
                       s: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    y = np.empty(rows, dtype=np.float64)
    mag = np.empty(rows, dtype=np.float64)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    lib().hyqo_gemv_q8_bruteforce(dtype, _p(w), rows, cols, _p(q), _p(s), _p(y), _p(mag))
    return y, mag


def dot(a: np.ndarray, b: np.ndarray) -> float:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return lib().hyqo_dot(_p(a), _p(b), a.size)


def dot_scalar(a: np.ndarray, b: np.ndarray) -> float:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return lib().hyqo_dot_scalar(_p(a), _p(b), a.size)


def row_dot_f32(dtype: int, row: np.ndarray, cols: int, x: np.ndarray) -> float:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().hyqo_row_dot_f32(dtype, _p(row), cols, _p(x))


def matmul(dtype: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray, batch: int,
           threads: int = 0) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(batch * rows, dtype=np.float32)
    rc = lib().hyqo_matmul(dtype, _p(w), rows, cols, _p(x), batch, _p(y), threads)
    if rc != 0:
        raise ValueError("matmul: invalid shape")
    return y.reshape(batch, rows)


def gate_up_silu(dtype: int, gate: np.ndarray, up: np.ndarray, rows: int, cols: int,
                 x: np.ndarray, threads: int = 0) -> np.ndarray:
    y = np.empty(rows, dtype=np.float32)
    gate = np.ascontiguousarray(gate, dtype=np.uint8)
    up = np.ascontiguousarray(up, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    rc = lib().hyqo_gate_up_silu(dtype, _p(gate), _p(up), rows, cols, _p(x), _p(y), threads)
    if rc != 0:
        raise ValueError("gate_up_silu: invalid shape")
    return y


def matmul_f64(dtype: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray,
               batch: int) -> tuple[np.ndarray, np.ndarray]:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(batch * rows, dtype=np.float64)
    mag = np.empty(batch * rows, dtype=np.float64)
    lib().hyqo_matmul_f64(dtype, _p(w), rows, cols, _p(x), batch, _p(y), _p(mag))
    return y.reshape(batch, rows), mag.reshape(batch, rows)


def route(logits: np.ndarray, bias: np.ndarray, used: int, normalize: bool,
          scale: float) -> list[tuple[int, float]]:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    bias = np.ascontiguousarray(bias, dtype=np.float32)
    idx = np.empty(used, dtype=np.int32)
    w = np.empty(used, dtype=np.float32)
    lib().hyqo_route(_p(logits), _p(bias), logits.size, used, int(normalize), scale,
                     _p(idx), _p(w))
    return [(int(i), float(v)) for i, v in zip(idx, w)]


def moe_experts(dtype_gate: int, dtype_down: int, gate: np.ndarray, up: np.ndarray,
                down: np.ndarray, experts: int, hidden: int, mid: int, x: np.ndarray,
                pairs_token: np.ndarray, pairs_expert: np.ndarray, pairs_weight: np.ndarray,
                out: np.ndarray, threads: int = 0) -> np.ndarray:
    gate = np.ascontiguousarray(gate, dtype=np.uint8)
    up = np.ascontiguousarray(up, dtype=np.uint8)
    down = np.ascontiguousarray(down, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    pt = np.ascontiguousarray(pairs_token, dtype=np.int32)
    pe = np.ascontiguousarray(pairs_expert, dtype=np.int32)
    pw = np.ascontiguousarray(pairs_weight, dtype=np.float32)
    out = np.ascontiguousarray(out, dtype=np.float32).copy()
    tokens = x.size // hidden
    lib().hyqo_moe_experts(dtype_gate, dtype_down, _p(gate), _p(up), _p(down), experts, hidden,
                           mid, _p(x), tokens, _p(pt), _p(pe), _p(pw), pt.size, _p(out),
                           threads)
    return out


class _Model(ctypes.Structure):
    _fields_ = [("layers", ctypes.c_int), ("hidden", ctypes.c_int), ("heads", ctypes.c_int),
                ("kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("ffn", ctypes.c_int),
                ("vocab", ctypes.c_int), ("rope_base", ctypes.c_float),
                ("eps", ctypes.c_float), ("dtype_linear", ctypes.c_int),
                ("dtype_embed", ctypes.c_int), ("dtype_down", ctypes.c_int), ("embed", P), ("output", P), ("output_norm", P),
                ("wq", P), ("wk", P), ("wv", P), ("wo", P), ("wgate", P), ("wup", P),
                ("wdown", P), ("attn_norm", P), ("ffn_norm", P), ("q_norm", P),
                ("k_norm", P), ("arch", ctypes.c_int), ("moe", P)]


# Q8 stages of the int8 path (oracle/hyq_oracle_step.h: hyqo_q8_tap)
STAGE_ATTN_IN, STAGE_OUT_IN, STAGE_FFN_IN, STAGE_DOWN_IN, STAGE_EXPERT_DOWN_IN = range(5)


class _Tap(ctypes.Structure):
    _fields_ = [("stride", SZ), ("own_x", P), ("own_q", P), ("own_s", P), ("use_q", P),
                ("use_s", P)]


class Q8Tap:
    """The oracle's own quantized inputs stage by stage (x, q, s: [stages,
    stride], [stages, stride], [stages, stride / 256]) and, for the stages in
    `use` ({stage: (codes, scales, ...)}), the codes and scales that replace
    them in the products."""

    def __init__(self, stages: int, width: int, use: dict | None = None, required=()):
        self.stride = (width + 255) // 256 * 256
        self.x = np.zeros((stages, self.stride), np.float32)
        self.q = np.zeros((stages, self.stride), np.int8)
        self.s = np.zeros((stages, self.stride // 256), np.float32)
        self.use_q = np.zeros((stages, self.stride), np.int8)
        self.use_s = np.zeros((stages, self.stride // 256), np.float32)
        # the C tap replaces every stage the run reaches, or none
        if use is not None and not set(required) <= set(use):
            raise ValueError("Q8Tap: codes for stages %s are missing"
                             % sorted(set(required) - set(use)))
        self._uses = bool(use)
        for st, rec in (use or {}).items():
            q, sc = rec[0], rec[1]
            self.use_q[st, :q.size] = q
            self.use_s[st, :sc.size] = sc
        self.st = _Tap(self.stride, _p(self.x), _p(self.q), _p(self.s),
                       _p(self.use_q) if self._uses else None,
                       _p(self.use_s) if self._uses else None)

    def own(self, stage: int, n: int):
        """The oracle's input, codes and scales of one stage's n values."""
        return self.x[stage, :n], self.q[stage, :n], self.s[stage, :(n + 255) // 256]


def moe_forward_tap(e: dict, hidden: int, x: np.ndarray, use: dict | None = None,
                    threads: int = 0):
    """Moe::forward of one row on the int8 path with its Q8 stages (FFN_IN,
    DOWN_IN, EXPERT_DOWN_IN + j) recorded and, with `use`, replaced."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.empty(hidden, np.float32)
    st = moe_struct(e)
    tap = Q8Tap(STAGE_EXPERT_DOWN_IN + e["used"], max(hidden, e["mid"], e["shared_mid"]), use,
                [STAGE_FFN_IN, STAGE_DOWN_IN] +
                [STAGE_EXPERT_DOWN_IN + j for j in range(e["used"])])
    lib().hyqo_moe_forward_tap(ctypes.byref(st), hidden, _p(x), _p(out), threads,
                               ctypes.byref(tap.st))
    return out, tap


class _Moe(ctypes.Structure):
    _fields_ = [("experts", ctypes.c_int), ("used", ctypes.c_int), ("mid", ctypes.c_int),
                ("shared_mid", ctypes.c_int), ("normalize", ctypes.c_int),
                ("scale", ctypes.c_float), ("dtype_gate", ctypes.c_int),
                ("dtype_down", ctypes.c_int), ("dtype_shared", ctypes.c_int),
                ("dtype_shared_down", ctypes.c_int), ("router", P), ("bias", P), ("gate", P),
                ("up", P), ("down", P), ("sgate", P), ("sup", P), ("sdown", P)]


def moe_struct(e: dict) -> _Moe:
    """The oracle's hyqo_moe for a synthetic MoE FFN (tests/synth.py)."""
    return _Moe(e["experts"], e["used"], e["mid"], e["shared_mid"], int(e["normalize"]),
                e["scale"], e["dtype_gate"], e["dtype_down"], e["dtype_shared"],
                e["dtype_shared_down"], _p(e["router"]), _p(e["bias"]), _p(e["gate"]),
                _p(e["up"]), _p(e["down"]), _p(e["sgate"]), _p(e["sup"]), _p(e["sdown"]))


def moe_forward(e: dict, hidden: int, x: np.ndarray, n: int, int8_path: bool,
                threads: int = 0) -> np.ndarray:
    """Moe::forward (src/model.rs:687-726) of n rows."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(n * hidden, np.float32)
    st = moe_struct(e)
    lib().hyqo_moe_forward(ctypes.byref(st), hidden, _p(x), n, _p(out), int(int8_path), threads)
    return out.reshape(n, hidden)


class DenseOracle:
    """Model::forward_into batch 1 on the CPU (oracle/hyq_oracle_step.c) over a
    synthetic model dict (tests/synth.py:make_dense_model)."""

    def __init__(self, model: dict):
        self.model = model
        c = model["cfg"]
        L = model["layers"]
        self._arrays = []

        def ptrs(key):
            arr = (P * len(L))(*[_p(layer[key]) if key in layer else None for layer in L])
            self._arrays.append(arr)
            return ctypes.cast(arr, P)

        self._moe = [moe_struct(layer["moe"]) if "moe" in layer else None for layer in L]
        moe_arr = (P * len(L))(*[ctypes.addressof(m) if m is not None else None
                                 for m in self._moe])
        self._arrays.append(moe_arr)

        self.m = _Model(c["layers"], c["hidden"], c["heads"], c["kv_heads"], c["head_dim"],
                        c["ffn"], c["vocab"], c["rope_base"], c["rms_eps"], model["linear"],
                        model["embed_dtype"], model.get("down_dtype", model["linear"]),
                        _p(model["embed"]),
                        _p(model["output"]) if "output" in model else None,
                        _p(model["output_norm"]),
                        ptrs("q"), ptrs("k"), ptrs("v"), ptrs("o"), ptrs("gate"), ptrs("up"),
                        ptrs("down"), ptrs("attn_norm"), ptrs("ffn_norm"), ptrs("q_norm"),
                        ptrs("k_norm"), model.get("arch", 0), ctypes.cast(moe_arr, P))

    def step(self, kcache: np.ndarray, vcache: np.ndarray, pos: int, token: int,
             int8_path: bool, threads: int = 0) -> np.ndarray:
        assert kcache.flags["C_CONTIGUOUS"] and vcache.flags["C_CONTIGUOUS"]
        ctx = kcache.shape[1]
        logits = np.empty(self.model["cfg"]["vocab"], np.float32)
        rc = lib().hyqo_decode_step(ctypes.byref(self.m), _p(kcache), _p(vcache), ctx, pos,
                                    token, int(int8_path), _p(logits), threads)
        if rc != 0:
            raise ValueError("decode_step: bad position or token")
        return logits

    def layer(self, l: int, hidden: np.ndarray, kc: np.ndarray, vc: np.ndarray, pos: int,
              int8_path: bool, threads: int = 0) -> np.ndarray:
        """One layer of the batch-1 step on a copy of `hidden` [H], with that
        layer's caches kc/vc [ctx, kv_heads*head_dim] (row `pos` written)."""
        h = np.ascontiguousarray(hidden, np.float32).copy()
        assert kc.flags["C_CONTIGUOUS"] and vc.flags["C_CONTIGUOUS"]
        rc = lib().hyqo_layer_step(ctypes.byref(self.m), l, _p(h), _p(kc), _p(vc),
                                   kc.shape[0], pos, int(int8_path), threads)
        if rc != 0:
            raise ValueError("layer_step: bad layer or position")
        return h

    def stages(self, l: int) -> list[int]:
        """Widths of layer l's Q8 stages (STAGE_*), in stage order."""
        c = self.model["cfg"]
        layer = self.model["layers"][l]
        w = [c["hidden"], c["heads"] * c["head_dim"], c["hidden"]]
        if "moe" in layer:
            e = layer["moe"]
            return w + [e["shared_mid"]] + [e["mid"]] * e["used"]
        return w + [c["ffn"]]

    def layer_tap(self, l: int, hidden: np.ndarray, kc: np.ndarray, vc: np.ndarray, pos: int,
                  use: dict | None = None, threads: int = 0):
        """layer() on the int8 path with the Q8 stages recorded and, with
        `use`, replaced: (output row, Q8Tap)."""
        h = np.ascontiguousarray(hidden, np.float32).copy()
        assert kc.flags["C_CONTIGUOUS"] and vc.flags["C_CONTIGUOUS"]
        widths = self.stages(l)
        tap = Q8Tap(len(widths), max(widths), use, range(len(widths)))
        rc = lib().hyqo_layer_step_tap(ctypes.byref(self.m), l, _p(h), _p(kc), _p(vc),
                                       kc.shape[0], pos, threads, ctypes.byref(tap.st))
        if rc != 0:
            raise ValueError("layer_step: bad layer or position")
        return h, tap

    def output_tap(self, hidden: np.ndarray, use: dict | None = None, threads: int = 0):
        """output() on the int8 path with its one Q8 stage (STAGE_ATTN_IN)
        recorded and, with `use`, replaced: (logits, Q8Tap)."""
        h = np.ascontiguousarray(hidden, np.float32).copy()
        logits = np.empty(self.model["cfg"]["vocab"], np.float32)
        tap = Q8Tap(1, self.model["cfg"]["hidden"], use, [STAGE_ATTN_IN])
        lib().hyqo_output_logits_tap(ctypes.byref(self.m), _p(h), _p(logits), threads,
                                     ctypes.byref(tap.st))
        return logits, tap

    def prefill_layer(self, l: int, hidden: np.ndarray, kc: np.ndarray, vc: np.ndarray,
                      pos: int, threads: int = 0) -> np.ndarray:
        """One layer of the batch-n arm on a copy of `hidden` [n, H]."""
        h = np.ascontiguousarray(hidden, np.float32).copy()
        n = h.size // self.model["cfg"]["hidden"]
        rc = lib().hyqo_prefill_layer(ctypes.byref(self.m), l, _p(h), _p(kc), _p(vc),
                                      kc.shape[0], pos, n, threads)
        if rc != 0:
            raise ValueError("prefill_layer: bad layer, rows or position")
        return h

    def output(self, hidden: np.ndarray, int8_path: bool, threads: int = 0) -> np.ndarray:
        """Output norm + output matmul of one hidden row."""
        h = np.ascontiguousarray(hidden, np.float32).copy()
        logits = np.empty(self.model["cfg"]["vocab"], np.float32)
        lib().hyqo_output_logits(ctypes.byref(self.m), _p(h), int(int8_path), _p(logits),
                                 threads)
        return logits

    def prefill(self, kcache: np.ndarray, vcache: np.ndarray, pos: int, tokens,
                int8_path: bool, threads: int = 0, chunk: int = 256) -> np.ndarray:
        """Model::prefill_into (src/model.rs:630-646): chunks of `chunk` tokens
        through forward_into at batch n; the last chunk's logits."""
        assert kcache.flags["C_CONTIGUOUS"] and vcache.flags["C_CONTIGUOUS"]
        toks = np.ascontiguousarray(tokens, np.int32)
        if toks.size == 0 or pos + toks.size > kcache.shape[1]:
            raise ValueError("prompt is empty or exceeds the context limit")
        logits = np.empty(self.model["cfg"]["vocab"], np.float32)
        for s in range(0, toks.size, chunk):
            part = toks[s:s + chunk]
            rc = lib().hyqo_prefill_chunk(ctypes.byref(self.m), _p(kcache), _p(vcache),
                                          kcache.shape[1], pos + s, _p(part), part.size,
                                          int(int8_path), _p(logits), threads)
            if rc != 0:
                raise ValueError("prefill_chunk: bad position or token")
        return logits
