"""Python binding of libhyq (include/hyq.h): MI355X quantized matmuls for hy-mt-rs.

Mirrors the reference's quantized-tensor interface (src/quant.rs):
``Weight.matmul``, ``Weight.gemv_qkv``, ``Weight.matmul_gate_up_silu``,
``Weight.expert``, ``Weight.row``, ``decode`` and the int8 ``Q8`` buffers,
with the same argument meanings and the same failures (ValueError where the
reference's ``ensure!`` fails). Every call runs the HIP kernels of libhyq.so;
there is no CPU fallback: importing without the built library, or calling
without a GPU, raises.
"""
from __future__ import annotations

import ctypes
import weakref
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhyq.so")

F32, F16, Q8_0, Q4_K, Q6_K, Q2_0C, STQ1_0 = 0, 1, 8, 12, 14, 40, 42
DTYPES = {"F32": F32, "F16": F16, "Q8_0": Q8_0, "Q4_K": Q4_K, "Q6_K": Q6_K,
          "Q2_0C": Q2_0C, "STQ1_0": STQ1_0}
OK, EINVAL, EDTYPE, EDEVICE, ENOMEM = 0, -1, -2, -3, -4

# Every exported symbol of include/hyq.h with its ctypes signature.
P = ctypes.c_void_p
SZ = ctypes.c_size_t
I = ctypes.c_int
SIGNATURES = {
    "hyq_last_error": (ctypes.c_char_p, []),
    "hyq_block_len": (I, [I]),
    "hyq_block_bytes": (I, [I]),
    "hyq_ctx_create": (I, [I, ctypes.POINTER(P)]),
    "hyq_ctx_destroy": (None, [P]),
    "hyq_ctx_stream": (P, [P]),
    "hyq_sync": (I, [P]),
    "hyq_ctx_set_q8_trace": (I, [P, P, SZ]),
    "hyq_ctx_q8_trace_records": (I, [P, P, SZ, P, P]),
    "hyq_device_alloc": (I, [P, SZ, ctypes.POINTER(P)]),
    "hyq_device_free": (I, [P, P]),
    "hyq_memcpy_h2d": (I, [P, P, P, SZ]),
    "hyq_memcpy_d2h": (I, [P, P, P, SZ]),
    "hyq_memcpy_d2d": (I, [P, P, P, SZ]),
    "hyq_weight_upload": (I, [P, I, P, SZ, P, I, ctypes.POINTER(P)]),
    "hyq_weight_expert": (I, [P, SZ, ctypes.POINTER(P)]),
    "hyq_weight_release": (None, [P]),
    "hyq_weight_info": (I, [P, ctypes.POINTER(I), P, ctypes.POINTER(I)]),
    "hyq_matmul": (I, [P, P, P, SZ, P]),
    "hyq_gemv_qkv": (I, [P, P, P, P, P, P, P, P]),
    "hyq_gate_up_silu": (I, [P, P, P, P, P]),
    "hyq_decode": (I, [P, I, P, SZ, P, SZ]),
    "hyq_weight_row": (I, [P, P, SZ, P, SZ]),
    "hyq_q8_create": (I, [P, SZ, ctypes.POINTER(P)]),
    "hyq_q8_release": (None, [P]),
    "hyq_q8_buffers": (I, [P, ctypes.POINTER(P), ctypes.POINTER(P), ctypes.POINTER(SZ)]),
    "hyq_quantize_q8_d": (I, [P, P, SZ, P]),
    "hyq_gemv_q8_d": (I, [P, P, P, P, P]),
    "hyq_gemv_qkv_q8_d": (I, [P, P, P, P, P, P, P, P]),
    "hyq_gate_up_silu_q8_d": (I, [P, P, P, P, P]),
    "hyq_isums_per_row": (I, [I, SZ]),
    "hyq_gemv_isums_d": (I, [P, P, P, P]),
    "hyq_matmul_d": (I, [P, P, P, SZ, P]),
    "hyq_matmul_noalloc_d": (I, [P, P, P, SZ, P]),
    "hyq_hbm_read_d": (I, [P, P, SZ, I, P]),
    "hyq_mfma_stream_d": (I, [P, I, I, P]),
    "hyq_dequant_rows_d": (I, [P, P, SZ, SZ, P]),
    "hyq_moe_scratch_bytes": (SZ, [SZ, SZ, SZ, SZ, SZ]),
    "hyq_moe_experts_d": (I, [P, P, P, P, P, SZ, P, P, P, SZ, P, SZ, P]),
    "hyq_moe_experts": (I, [P, P, P, P, P, SZ, P, P, P, SZ, P]),
    "hyq_moe_shared_experts_d": (I, [P, P, P, P, P, P, SZ, P, P, P, SZ, P, SZ, P]),
    "hyq_decode_d": (I, [P, I, P, SZ, P, SZ]),
    "hyq_embed_row_d": (I, [P, P, P, P]),
    "hyq_rms_norm_q8_d": (I, [P, P, P, SZ, ctypes.c_float, P, P]),
    "hyq_rope_norm_append_d": (I, [P, P, P, P, P, P, P, P, SZ, SZ, SZ, ctypes.c_float, P, P]),
    "hyq_attention_scratch_floats": (SZ, [SZ, SZ]),
    "hyq_attention_d": (I, [P, P, P, P, P, SZ, SZ, SZ, SZ, P, P, P]),
    "hyq_attention_rope_d": (I, [P, P, P, P, P, P, P, P, SZ, SZ, SZ, SZ, ctypes.c_float, I, P, P,
                                 P, P]),
    "hyq_attention_rows_scratch_floats": (SZ, [SZ, SZ, SZ]),
    "hyq_attention_rows_d": (I, [P, P, P, P, P, SZ, SZ, SZ, SZ, SZ, P, P]),
    "hyq_argmax_d": (I, [P, P, SZ, P, P]),
    "hyq_dense_create": (I, [P, P, SZ, ctypes.POINTER(P)]),
    "hyq_dense_destroy": (None, [P]),
    "hyq_dense_set_layer": (I, [P, I, P, P, P, P, P, P, P, P, P, P, P]),
    "hyq_dense_set_output": (I, [P, P, P, P]),
    "hyq_dense_load_kv": (I, [P, I, SZ, P, P]),
    "hyq_dense_set_position": (I, [P, SZ]),
    "hyq_dense_get_position": (I, [P, ctypes.POINTER(SZ)]),
    "hyq_dense_forward": (I, [P, ctypes.c_int32, P, P]),
    "hyq_dense_prefill": (I, [P, P, SZ, P, P]),
    "hyq_dense_read_kv": (I, [P, I, SZ, P, P]),
    "hyq_dense_set_prefill_rows": (I, [P, SZ]),
    "hyq_dense_set_trace": (I, [P, P, SZ]),
    "hyq_dense_set_architecture": (I, [P, I]),
    "hyq_dense_set_moe": (I, [P, I, P, P, P, P, P, P, P, P, P]),
    "hyq_moe_route_d": (I, [P, P, P, SZ, SZ, SZ, I, ctypes.c_float, P, P, P]),
    "hyq_moe_forward_scratch_bytes": (SZ, [P, SZ, SZ]),
    "hyq_moe_forward_d": (I, [P, P, P, P, P, P, P, P, P, P, P, SZ, P, SZ, P]),
    "hyq_dense_generate": (I, [P, ctypes.c_int32, SZ, I, P]),
    "hyq_gguf_open": (I, [ctypes.c_char_p, I, ctypes.POINTER(P)]),
    "hyq_gguf_open_bytes": (I, [P, SZ, I, ctypes.POINTER(P)]),
    "hyq_gguf_close": (None, [P]),
    "hyq_gguf_profile": (I, [P]),
    "hyq_gguf_byte_len": (SZ, [P]),
    "hyq_gguf_bytes": (P, [P]),
    "hyq_gguf_tensor_count": (SZ, [P]),
    "hyq_gguf_tensor_at": (I, [P, SZ, P]),
    "hyq_gguf_find_tensor": (I, [P, ctypes.c_char_p, P]),
    "hyq_gguf_meta_u64": (I, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]),
    "hyq_gguf_meta_f64": (I, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
    "hyq_gguf_meta_bool": (I, [P, ctypes.c_char_p, ctypes.POINTER(I)]),
    "hyq_gguf_meta_str": (I, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p),
                              ctypes.POINTER(SZ)]),
    "hyq_gguf_meta_array": (I, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32),
                                ctypes.POINTER(ctypes.c_uint64)]),
    "hyq_gguf_upload": (I, [P, P, ctypes.c_char_p, ctypes.POINTER(P)]),
    "hyq_gguf_read_f32": (I, [P, P, ctypes.c_char_p, P, SZ]),
    "hyq_sha256": (I, [P, SZ, P]),
    "hyq_dense_from_gguf": (I, [P, P, SZ, ctypes.POINTER(P)]),
}

PROFILE_AUTO, PROFILE_STANDARD, PROFILE_TENCENT_Q2_0C, PROFILE_TENCENT_STQ1 = 0, 1, 2, 3
PROFILES = {"auto": PROFILE_AUTO, "standard": PROFILE_STANDARD,
            "tencent-q2-0c": PROFILE_TENCENT_Q2_0C, "tencent-stq1": PROFILE_TENCENT_STQ1}


class GgufTensor(ctypes.Structure):
    """hyq_gguf_tensor: TensorInfo (src/gguf.rs:28-38)."""
    _fields_ = [("name", ctypes.c_char_p), ("dims", ctypes.c_uint64 * 4), ("rank", I),
                ("type_id", ctypes.c_uint32), ("dtype", I), ("offset", ctypes.c_uint64),
                ("byte_len", ctypes.c_uint64)]


class DenseConfig(ctypes.Structure):
    """hyq_dense_config: the Config fields the decode step uses (src/model.rs:29-40)."""
    _fields_ = [("layers", I), ("hidden", I), ("heads", I), ("kv_heads", I),
                ("head_dim", I), ("ffn", I), ("vocab", I), ("rope_base", ctypes.c_float),
                ("rms_eps", ctypes.c_float)]

_lib = None


def lib() -> ctypes.CDLL:
    """Load libhyq.so (built by build.py / __graft_entry__.build())."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run hy-mt-rs_amd/build.py first")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class HyqError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"hyq error {code}: {msg}")
        self.code = code


def check(rc: int) -> None:
    if rc == OK:
        return
    msg = lib().hyq_last_error().decode(errors="replace")
    if rc in (EINVAL, EDTYPE):
        raise ValueError(f"hyq error {rc}: {msg}")
    raise HyqError(rc, msg)


def _ptr(a: np.ndarray) -> int:
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C-contiguous")
    return a.ctypes.data


def row_bytes(dtype: int, cols: int) -> int:
    return cols // lib().hyq_block_len(dtype) * lib().hyq_block_bytes(dtype)


class Context:
    """One device and one HIP stream (include/hyq.h: hyq_ctx)."""

    def __init__(self, device: int = 0):
        h = P()
        check(lib().hyq_ctx_create(device, ctypes.byref(h)))
        self.handle = h.value
        self.device = device
        # objects that use the context's stream (decoders): closed first
        self._dependents = weakref.WeakSet()
        # device buffers allocated through the context: freed by close(), so
        # that none is left to the HIP runtime's own teardown at process exit
        self._buffers = weakref.WeakSet()
        self._q8trace = None

    @property
    def stream(self) -> int:
        return lib().hyq_ctx_stream(self.handle)

    def sync(self) -> None:
        check(lib().hyq_sync(self.handle))

    def close(self) -> None:
        """Closes the decoders on the context, synchronises its stream, frees
        every device buffer allocated through it, then destroys it."""
        if self.handle:
            for d in list(self._dependents):
                d.close()
            check(lib().hyq_sync(self.handle))
            if self._q8trace is not None:
                check(lib().hyq_ctx_set_q8_trace(self.handle, None, 0))
            for b in list(self._buffers):
                b.free()
            self._q8trace = None
            lib().hyq_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def decode(self, dtype: int, data, n: int | None = None) -> np.ndarray:
        """decode (src/quant.rs:1066) on the device."""
        buf = np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8)
                                   if not isinstance(data, np.ndarray) else data, np.uint8)
        if n is None:
            n = buf.size // lib().hyq_block_bytes(dtype) * lib().hyq_block_len(dtype)
        out = np.empty(n, np.float32)
        check(lib().hyq_decode(self.handle, dtype, _ptr(buf), buf.size, _ptr(out), n))
        return out

    def array(self, a: np.ndarray) -> "DeviceArray":
        """A device copy of a numpy array."""
        return DeviceArray.from_host(self, a)

    def empty(self, shape, dtype) -> "DeviceArray":
        return DeviceArray(self, shape, dtype)

    def upload(self, dtype: int, data: np.ndarray, dims: tuple[int, ...]) -> "Weight":
        return Weight.upload(self, dtype, data, dims)

    def q8(self, n: int) -> "Q8":
        return Q8(self, n)

    def set_q8_trace(self, nbytes: int | None) -> None:
        """Record the int8 codes and scales the decode path's launches form
        (hyq_ctx_set_q8_trace) into a device buffer of `nbytes`; None stops
        recording. Each call starts an empty record list."""
        if not nbytes:
            check(lib().hyq_ctx_set_q8_trace(self.handle, None, 0))
            self._q8trace = None
            return
        self._q8trace = self.empty(nbytes, np.uint8)
        check(lib().hyq_ctx_set_q8_trace(self.handle, self._q8trace.ptr, nbytes))

    def clear_q8_trace(self) -> None:
        """Empty the record list, keeping the buffer."""
        check(lib().hyq_ctx_set_q8_trace(self.handle, self._q8trace.ptr, self._q8trace.nbytes))

    def q8_trace(self) -> list:
        """(codes int8 [n], scales f32 [n / 256], values f32 [n]) of every
        record since the list was emptied, in launch order: the codes and
        scales a launch formed and the f32 values it quantized."""
        count, dropped = ctypes.c_size_t(), ctypes.c_size_t()
        check(lib().hyq_ctx_q8_trace_records(self.handle, None, 0, ctypes.byref(count),
                                             ctypes.byref(dropped)))
        if dropped.value:
            raise RuntimeError(f"q8 trace: {dropped.value} records did not fit")
        pairs = (ctypes.c_size_t * (2 * count.value + 2))()
        check(lib().hyq_ctx_q8_trace_records(self.handle, pairs, count.value,
                                             ctypes.byref(count), None))
        self.sync()
        raw = self._q8trace.numpy()
        out = []
        for i in range(count.value):
            o, n = pairs[2 * i], pairs[2 * i + 1]
            xo = o + (n + n // 64 + 255) // 256 * 256
            out.append((raw[o:o + n].view(np.int8).copy(),
                        raw[o + n:o + n + n // 64].view(np.float32).copy(),
                        raw[xo:xo + 4 * n].view(np.float32).copy()))
        return out


class DeviceArray:
    """A device buffer owned through the C ABI (hyq_device_alloc)."""

    def __init__(self, ctx: Context, shape, dtype):
        self.ctx = ctx
        self.shape = tuple(shape) if isinstance(shape, (tuple, list)) else (int(shape),)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        h = P()
        check(lib().hyq_device_alloc(ctx.handle, self.nbytes, ctypes.byref(h)))
        self.ptr = h.value
        ctx._buffers.add(self)

    @classmethod
    def from_host(cls, ctx: Context, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(ctx, a.shape, a.dtype)
        d.copy_from(a)
        return d

    def copy_from(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, self.dtype)
        if a.nbytes != self.nbytes:
            raise ValueError("size mismatch")
        check(lib().hyq_memcpy_h2d(self.ctx.handle, self.ptr, _ptr(a), self.nbytes))

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(lib().hyq_memcpy_d2h(self.ctx.handle, _ptr(out), self.ptr, self.nbytes))
        return out

    def free(self) -> None:
        if self.ptr and self.ctx.handle:
            lib().hyq_device_free(self.ctx.handle, self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Weight:
    """A packed quantized tensor on the device (src/quant.rs:65-154)."""

    def __init__(self, ctx: Context, handle: int, parent: "Weight | None" = None):
        self.ctx = ctx
        self.handle = handle
        self._parent = parent
        dt = I()
        dims = (ctypes.c_uint64 * 3)()
        rank = I()
        check(lib().hyq_weight_info(handle, ctypes.byref(dt), ctypes.cast(dims, P),
                                    ctypes.byref(rank)))
        self.dtype = dt.value
        self.rank = rank.value
        self.dims = tuple(int(d) for d in dims[:self.rank])

    @classmethod
    def upload(cls, ctx: Context, dtype: int, data: np.ndarray, dims) -> "Weight":
        buf = np.ascontiguousarray(data, np.uint8)
        d = (ctypes.c_uint64 * 3)(*[int(v) for v in dims], *([1] * (3 - len(dims))))
        h = P()
        check(lib().hyq_weight_upload(ctx.handle, dtype, _ptr(buf), buf.size, ctypes.cast(d, P),
                                      len(dims), ctypes.byref(h)))
        return cls(ctx, h.value)

    def shape(self) -> tuple[int, ...]:
        return self.dims

    @property
    def cols(self) -> int:
        return self.dims[0]

    @property
    def rows(self) -> int:
        return self.dims[1]

    def release(self) -> None:
        if self.handle:
            lib().hyq_weight_release(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def expert(self, index: int) -> "Weight":
        """Weight::expert (src/quant.rs:144-154): a no-copy view."""
        h = P()
        check(lib().hyq_weight_expert(self.handle, index, ctypes.byref(h)))
        return Weight(self.ctx, h.value, parent=self)

    def matmul(self, x: np.ndarray, batch: int) -> np.ndarray:
        """Weight::matmul (src/quant.rs:159): x [batch*cols] -> [batch*rows]."""
        x = np.ascontiguousarray(x, np.float32)
        if x.size != batch * self.cols:
            raise ValueError("invalid activation shape")
        y = np.empty(batch * self.rows, np.float32)
        check(lib().hyq_matmul(self.ctx.handle, self.handle, _ptr(x), batch, _ptr(y)))
        return y

    @staticmethod
    def gemv_qkv(q: "Weight", k: "Weight", v: "Weight", x: np.ndarray):
        """Weight::gemv_qkv (src/quant.rs:658)."""
        x = np.ascontiguousarray(x, np.float32)
        if x.size != q.cols:
            raise ValueError("invalid activation shape for qkv")
        yq, yk, yv = (np.empty(w.rows, np.float32) for w in (q, k, v))
        check(lib().hyq_gemv_qkv(q.ctx.handle, q.handle, k.handle, v.handle, _ptr(x), _ptr(yq),
                                 _ptr(yk), _ptr(yv)))
        return yq, yk, yv

    def matmul_gate_up_silu(self, up: "Weight", x: np.ndarray) -> np.ndarray:
        """Weight::matmul_gate_up_silu (src/quant.rs:724)."""
        x = np.ascontiguousarray(x, np.float32)
        if x.size != self.cols:
            raise ValueError("invalid activation shape for gate_up_silu")
        y = np.empty(self.rows, np.float32)
        check(lib().hyq_gate_up_silu(self.ctx.handle, self.handle, up.handle, _ptr(x), _ptr(y)))
        return y

    def row(self, index: int) -> np.ndarray:
        """Weight::row (src/quant.rs:106)."""
        out = np.empty(self.cols, np.float32)
        check(lib().hyq_weight_row(self.ctx.handle, self.handle, index, _ptr(out), out.size))
        return out


class Q8:
    """Device int8 activations with per-256 scales (src/quant.rs:861-941)."""

    def __init__(self, ctx: Context, n: int):
        self.ctx = ctx
        h = P()
        check(lib().hyq_q8_create(ctx.handle, n, ctypes.byref(h)))
        self.handle = h.value
        self.n = n
        q, s, nn = P(), P(), SZ()
        check(lib().hyq_q8_buffers(self.handle, ctypes.byref(q), ctypes.byref(s),
                                   ctypes.byref(nn)))
        self.values_ptr, self.scales_ptr = q.value, s.value

    def release(self) -> None:
        if self.handle:
            lib().hyq_q8_release(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def quantize_into(self, x_dev_ptr: int) -> None:
        check(lib().hyq_quantize_q8_d(self.ctx.handle, x_dev_ptr, self.n, self.handle))


def moe_experts(gate: "Weight", up: "Weight", down: "Weight", x: np.ndarray, tokens: int,
                pair_token, pair_expert, pair_weight, out: np.ndarray) -> np.ndarray:
    """Expert loop of Moe::forward (src/model.rs:699-725): returns ``out`` plus,
    per token and in ascending expert order, weight * DenseFfn_e(x[token]).
    ``out`` [tokens*hidden] is the seed (the shared expert's output)."""
    x = np.ascontiguousarray(x, np.float32)
    hidden = gate.dims[0]
    if x.size != tokens * hidden:
        raise ValueError("invalid activation shape")
    pt = np.ascontiguousarray(pair_token, np.int32)
    pe = np.ascontiguousarray(pair_expert, np.int32)
    pw = np.ascontiguousarray(pair_weight, np.float32)
    if not (pt.size == pe.size == pw.size):
        raise ValueError("routing lists differ in length")
    res = np.array(out, np.float32, copy=True).reshape(-1)
    if res.size != tokens * hidden:
        raise ValueError("invalid output shape")
    check(lib().hyq_moe_experts(gate.ctx.handle, gate.handle, up.handle, down.handle, _ptr(x),
                                tokens, _ptr(pt), _ptr(pe), _ptr(pw), pt.size, _ptr(res)))
    return res


def isums_per_row(dtype: int, cols: int) -> int:
    return lib().hyq_isums_per_row(dtype, cols)


ARCH_DENSE, ARCH_HYV3 = 0, 1


class MoeConfig(ctypes.Structure):
    """hyq_moe_config: the expert_* metadata of a HyV3 model."""
    _fields_ = [("experts", I), ("used", I), ("mid", I), ("shared_mid", I), ("normalize", I),
                ("scale", ctypes.c_float)]


class MoeFfn:
    """Moe::forward (src/model.rs:687-726) on the device: an F32 router, its
    selection bias, expert stacks (rank-3 ``Weight``s) and a shared expert."""

    def __init__(self, ctx: "Context", cfg: MoeConfig, router, bias, gate, up, down, sgate,
                 sup, sdown):
        self.ctx, self.cfg = ctx, cfg
        self.weights = (router, gate, up, down, sgate, sup, sdown)
        self.bias = ctx.array(np.ascontiguousarray(bias, np.float32))
        self.hidden = router.cols

    def forward_d(self, x_d: int, tokens: int, out_d: int) -> None:
        """hyq_moe_forward_d on device buffers x [tokens][hidden] -> out."""
        need = lib().hyq_moe_forward_scratch_bytes(ctypes.byref(self.cfg), self.hidden, tokens)
        if need == 0:
            raise ValueError("moe_forward: unsupported token count")
        scratch = self.ctx.empty(need, np.uint8)
        r, g, u, d, sg, su, sd = self.weights
        check(lib().hyq_moe_forward_d(self.ctx.handle, ctypes.byref(self.cfg), r.handle,
                                      self.bias.ptr, g.handle, u.handle, d.handle, sg.handle,
                                      su.handle, sd.handle, x_d, tokens, scratch.ptr, need,
                                      out_d))
        self.ctx.sync()

    def forward(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.hidden)
        xd = self.ctx.array(x)
        od = self.ctx.empty(x.size, np.float32)
        self.forward_d(xd.ptr, x.shape[0], od.ptr)
        return od.numpy().reshape(x.shape)


def moe_route(ctx: "Context", logits: np.ndarray, bias: np.ndarray, used: int, normalize: bool,
              scale: float):
    """route (src/model.rs:728-767) of logits [tokens][experts] on the
    device: (token, expert, weight) arrays, token-major, ascending experts."""
    logits = np.ascontiguousarray(logits, np.float32)
    tokens, experts = logits.shape
    ld, bd = ctx.array(logits), ctx.array(np.ascontiguousarray(bias, np.float32))
    pt = ctx.empty(tokens * used, np.int32)
    pe = ctx.empty(tokens * used, np.int32)
    pw = ctx.empty(tokens * used, np.float32)
    check(lib().hyq_moe_route_d(ctx.handle, ld.ptr, bd.ptr, tokens, experts, used,
                                int(normalize), scale, pt.ptr, pe.ptr, pw.ptr))
    return pt.numpy(), pe.numpy(), pw.numpy()


class DenseDecoder:
    """Batch-1 decode of the dense graph on the device (Model::forward_into,
    src/model.rs:374-546, plus greedy sampling). Weights are borrowed
    ``Weight`` objects; norm vectors are f32 numpy arrays."""

    def __init__(self, ctx: Context, cfg: DenseConfig, context: int):
        self.ctx = ctx
        self.cfg = cfg
        h = P()
        check(lib().hyq_dense_create(ctx.handle, ctypes.byref(cfg), context, ctypes.byref(h)))
        self.handle = h.value
        self._keep = []
        ctx._dependents.add(self)

    def close(self) -> None:
        # a decoder uses its context's stream: it goes first (Context.close)
        if self.handle and self.ctx.handle:
            lib().hyq_dense_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_layer(self, layer: int, q, k, v, o, gate, up, down, attn_norm, ffn_norm,
                  q_norm, k_norm) -> None:
        norms = [np.ascontiguousarray(a, np.float32) for a in (attn_norm, ffn_norm, q_norm,
                                                               k_norm)]
        h = lambda w: w.handle if w is not None else None
        check(lib().hyq_dense_set_layer(self.handle, layer, q.handle, k.handle, v.handle,
                                        o.handle, h(gate), h(up), h(down),
                                        *[_ptr(a) for a in norms]))
        self._keep.extend([q, k, v, o, gate, up, down])

    def set_architecture(self, arch: int) -> None:
        check(lib().hyq_dense_set_architecture(self.handle, arch))

    def set_moe(self, layer: int, ffn: MoeFfn) -> None:
        """The layer's FFN becomes ``ffn`` (Ffn::Moe)."""
        r, g, u, d, sg, su, sd = ffn.weights
        bias = ffn.bias.numpy()
        check(lib().hyq_dense_set_moe(self.handle, layer, ctypes.byref(ffn.cfg), r.handle,
                                      _ptr(bias), g.handle, u.handle, d.handle, sg.handle,
                                      su.handle, sd.handle))
        self._keep.append(ffn)

    def set_output(self, embedding, output, output_norm) -> None:
        on = np.ascontiguousarray(output_norm, np.float32)
        check(lib().hyq_dense_set_output(self.handle, embedding.handle, output.handle, _ptr(on)))
        self._keep.extend([embedding, output])

    def load_kv(self, layer: int, keys: np.ndarray, values: np.ndarray) -> None:
        keys = np.ascontiguousarray(keys, np.float32)
        values = np.ascontiguousarray(values, np.float32)
        kvw = self.cfg.kv_heads * self.cfg.head_dim
        if keys.size != values.size or keys.size % kvw:
            raise ValueError("keys/values must be [positions, kv_heads*head_dim]")
        check(lib().hyq_dense_load_kv(self.handle, layer, keys.size // kvw, _ptr(keys),
                                      _ptr(values)))

    @property
    def position(self) -> int:
        p = SZ()
        check(lib().hyq_dense_get_position(self.handle, ctypes.byref(p)))
        return p.value

    @position.setter
    def position(self, pos: int) -> None:
        check(lib().hyq_dense_set_position(self.handle, pos))

    def forward(self, token: int, want_logits: bool = True):
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        nxt = ctypes.c_int32()
        check(lib().hyq_dense_forward(self.handle, token,
                                      _ptr(logits) if logits is not None else None,
                                      ctypes.byref(nxt)))
        return logits, nxt.value

    def prefill(self, tokens, want_logits: bool = True):
        """Model::prefill_into (src/model.rs:630-646): the prompt through the
        batch > 1 forward pass; returns (last logits or None, greedy next
        token)."""
        toks = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        nxt = ctypes.c_int32()
        check(lib().hyq_dense_prefill(self.handle, _ptr(toks) if toks.size else None, toks.size,
                                      _ptr(logits) if logits is not None else None,
                                      ctypes.byref(nxt)))
        return logits, nxt.value

    @classmethod
    def from_gguf(cls, ctx: "Context", gguf: "Gguf", context: int) -> "DenseDecoder":
        """Model::from_gguf (src/model.rs:136-262, dense arm) + a session of
        `context` positions; the decoder owns the uploaded weights."""
        h = P()
        check(lib().hyq_dense_from_gguf(ctx.handle, gguf.handle, context, ctypes.byref(h)))
        self = cls.__new__(cls)
        self.ctx = ctx
        c = gguf
        self.cfg = DenseConfig(
            c.u64(f"{c.architecture}.block_count"), c.u64(f"{c.architecture}.embedding_length"),
            c.u64(f"{c.architecture}.attention.head_count"),
            c.u64(f"{c.architecture}.attention.head_count_kv"),
            c.u64(f"{c.architecture}.attention.key_length"),
            c.u64(f"{c.architecture}.feed_forward_length"), c.array_len("tokenizer.ggml.tokens"),
            c.f64(f"{c.architecture}.rope.freq_base"),
            c.f64(f"{c.architecture}.attention.layer_norm_rms_epsilon"))
        self.handle = h.value
        self._keep = [gguf]
        ctx._dependents.add(self)
        return self

    def set_prefill_rows(self, rows: int) -> None:
        """Tokens per device pass of prefill (results do not depend on it)."""
        check(lib().hyq_dense_set_prefill_rows(self.handle, rows))

    def set_trace(self, rows: int | None) -> None:
        """Record the hidden row after the embedding and after every layer
        (eager forward: one token; prefill: a pass of up to ``rows`` tokens);
        ``None`` stops recording. ``trace()`` reads the last record."""
        self._trace = None
        if rows is None:
            check(lib().hyq_dense_set_trace(self.handle, None, 0))
            return
        n = (self.cfg.layers + 1) * rows * self.cfg.hidden
        self._trace = self.ctx.empty(n, np.float32)
        check(lib().hyq_dense_set_trace(self.handle, self._trace.ptr, n))

    def trace(self, rows: int = 1) -> np.ndarray:
        """[layers + 1, rows, hidden] hidden rows of the last traced pass."""
        h = self.cfg.hidden
        t = self._trace.numpy()[:(self.cfg.layers + 1) * rows * h]
        return t.reshape(self.cfg.layers + 1, rows, h)

    def read_kv(self, layer: int, positions: int):
        """Cached keys and values [positions, kv_heads*head_dim] of one layer."""
        kvw = self.cfg.kv_heads * self.cfg.head_dim
        keys = np.empty((positions, kvw), np.float32)
        values = np.empty((positions, kvw), np.float32)
        check(lib().hyq_dense_read_kv(self.handle, layer, positions, _ptr(keys), _ptr(values)))
        return keys, values

    def generate(self, token: int, steps: int, use_graph: bool = True) -> np.ndarray:
        out = np.empty(steps, np.int32)
        check(lib().hyq_dense_generate(self.handle, token, steps, int(use_graph), _ptr(out)))
        return out


class Gguf:
    """A GGUF v3 file (Gguf::open, src/gguf.rs:50-210): validated like the
    reference, tensors by name, metadata accessors, uploads to the device.
    ``profile``: "auto", "standard", "tencent-q2-0c" or "tencent-stq1"."""

    def __init__(self, path=None, profile: str = "auto", data: bytes | None = None):
        if (path is None) == (data is None):
            raise ValueError("give a path or the file's bytes")
        h = P()
        pid = PROFILES[profile]
        if path is not None:
            check(lib().hyq_gguf_open(os.fsencode(path), pid, ctypes.byref(h)))
            self._buf = None
        else:
            self._buf = np.frombuffer(bytes(data), np.uint8)  # borrowed by the handle
            check(lib().hyq_gguf_open_bytes(self._buf.ctypes.data if self._buf.size else None,
                                            self._buf.size, pid, ctypes.byref(h)))
        self.handle = h.value

    def close(self) -> None:
        if self.handle:
            lib().hyq_gguf_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def profile(self) -> str:
        pid = lib().hyq_gguf_profile(self.handle)
        return {v: k for k, v in PROFILES.items()}[pid]

    @property
    def architecture(self) -> str:
        return self.string("general.architecture")

    def tensors(self) -> dict:
        """name -> dict(dims, type_id, dtype, offset, byte_len), in name order."""
        out = {}
        t = GgufTensor()
        for i in range(lib().hyq_gguf_tensor_count(self.handle)):
            check(lib().hyq_gguf_tensor_at(self.handle, i, ctypes.byref(t)))
            out[t.name.decode()] = dict(dims=list(t.dims[:t.rank]), type_id=t.type_id,
                                        dtype=t.dtype, offset=t.offset, byte_len=t.byte_len)
        return out

    def tensor_bytes(self, name: str) -> np.ndarray:
        t = GgufTensor()
        check(lib().hyq_gguf_find_tensor(self.handle, name.encode(), ctypes.byref(t)))
        base = lib().hyq_gguf_bytes(self.handle)
        return np.ctypeslib.as_array((ctypes.c_uint8 * t.byte_len).from_address(
            base + t.offset)).copy()

    def u64(self, key: str) -> int:
        v = ctypes.c_uint64()
        check(lib().hyq_gguf_meta_u64(self.handle, key.encode(), ctypes.byref(v)))
        return v.value

    def f64(self, key: str) -> float:
        v = ctypes.c_double()
        check(lib().hyq_gguf_meta_f64(self.handle, key.encode(), ctypes.byref(v)))
        return v.value

    def boolean(self, key: str) -> bool:
        v = I()
        check(lib().hyq_gguf_meta_bool(self.handle, key.encode(), ctypes.byref(v)))
        return bool(v.value)

    def string(self, key: str) -> str:
        p, n = ctypes.c_char_p(), SZ()
        check(lib().hyq_gguf_meta_str(self.handle, key.encode(), ctypes.byref(p),
                                      ctypes.byref(n)))
        return ctypes.string_at(p, n.value).decode()

    def array_len(self, key: str) -> int:
        et, n = ctypes.c_uint32(), ctypes.c_uint64()
        check(lib().hyq_gguf_meta_array(self.handle, key.encode(), ctypes.byref(et),
                                        ctypes.byref(n)))
        return n.value

    def upload(self, ctx: "Context", name: str) -> "Weight":
        """Gguf::tensor as a device weight (rank 2 or 3)."""
        h = P()
        check(lib().hyq_gguf_upload(ctx.handle, self.handle, name.encode(), ctypes.byref(h)))
        return Weight(ctx, h.value)

    def read_f32(self, ctx: "Context", name: str) -> np.ndarray:
        """Weight::to_vec of a tensor (norm vectors)."""
        n = int(np.prod(self.tensors()[name]["dims"]))
        out = np.empty(n, np.float32)
        check(lib().hyq_gguf_read_f32(ctx.handle, self.handle, name.encode(), _ptr(out), n))
        return out


def sha256(data: bytes) -> str:
    """SHA-256 hex digest computed by the library (the AUTO profile's check)."""
    buf = np.frombuffer(bytes(data), np.uint8)
    out = np.empty(32, np.uint8)
    check(lib().hyq_sha256(buf.ctypes.data if buf.size else None, buf.size, _ptr(out)))
    return out.tobytes().hex()
