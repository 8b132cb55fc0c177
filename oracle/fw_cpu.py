"""ctypes binding of the oracle (oracle/libfwcpu.so, the C restatement of
forword.c's forward).  TEST INFRASTRUCTURE: imported only by tests/, the smoke
check and the benchmark's CPU-baseline leg, always as the checker or the CPU
baseline, never on the product path."""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.environ.get("FW_CPU_LIB") or os.path.join(HERE, "libfwcpu.so")   # override: instrumented builds
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "forword.c_amd"))
import fwgpu  # noqa: E402  (struct layouts of the C ABI)

vp, sz, fp, u32p = C.c_void_p, C.c_size_t, C.POINTER(C.c_float), C.POINTER(C.c_uint32)
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} is not built (make -C oracle)")
        L = C.CDLL(LIB)
        s = fwgpu._sig
        s(L, "fwc_half_to_float", C.c_float, [C.c_uint16])
        s(L, "fwc_half_to_float_n", None, [vp, fp, sz])
        s(L, "fwc_dot_f32", C.c_float, [fp, fp, sz])
        s(L, "fwc_dequant", C.c_int, [vp, sz, C.c_uint32, fp, sz])
        s(L, "fwc_quant_matvec", C.c_int, [vp, sz, C.c_uint32, fp, fp, sz, sz])
        s(L, "fwc_rms_norm", None, [fp, fp, fp, sz, C.c_float])
        s(L, "fwc_rope_apply", None, [fp, sz, sz, sz, fp, fp, C.c_int])
        s(L, "fwc_softmax", None, [fp, sz])
        s(L, "fwc_silu", None, [fp, sz])
        s(L, "fwc_gelu", None, [fp, sz])
        s(L, "fwc_gelu_fast", None, [fp, sz])
        s(L, "fwc_argmax", C.c_uint32, [fp, sz])
        s(L, "fwc_attention_core", None, [fp, fp, fp, fp, sz, sz, sz, sz, fp])
        s(L, "fwc_tensor_matvec_f32", C.c_int, [fp, fp, fp, sz, sz])
        s(L, "fwc_set_threads", None, [C.c_int])
        s(L, "fwc_model_init", vp, [vp, sz, C.POINTER(fwgpu.TensorDesc), sz, C.POINTER(fwgpu.Config), sz,
                                    fp, fp])
        s(L, "fwc_model_free", None, [vp])
        s(L, "fwc_forward", fp, [vp, C.c_uint32, sz])
        s(L, "fwc_trace", fp, [vp])
        s(L, "fwc_kv_k", fp, [vp, sz, sz])
        s(L, "fwc_kv_v", fp, [vp, sz, sz])
        s(L, "fwc_generate_greedy", C.c_int, [vp, u32p, sz, sz, u32p])
        s(L, "fwc_sample", C.c_uint32, [fp, sz, u32p, sz, C.c_float, C.c_float, C.c_float,
                                        C.POINTER(C.c_uint64)])
        s(L, "fwc_generate_sampled", C.c_int, [vp, u32p, sz, sz, C.c_float, C.c_float, C.c_float, C.c_uint64,
                                               u32p])
        _lib = L
    return _lib


def _f(a):
    return a.ctypes.data_as(fp)


def set_threads(n: int):
    lib().fwc_set_threads(n)


def half_to_float(h: int) -> float:
    return lib().fwc_half_to_float(h)


def half_to_float_n(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.size, np.float32)
    lib().fwc_half_to_float_n(h.ctypes.data, _f(out), h.size)
    return out


def dot(a, b) -> np.float32:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return np.float32(lib().fwc_dot_f32(_f(a), _f(b), a.size))


def dequant(blocks: np.ndarray, ggml_type: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, np.uint8)
    n = blocks.size // fwgpu.BLOCK_BYTES[ggml_type] * fwgpu.BLOCK_VALUES[ggml_type]
    out = np.empty(n, np.float32)
    if lib().fwc_dequant(blocks.ctypes.data, blocks.size, ggml_type, _f(out), n) != 0:
        raise ValueError("fwc_dequant rejected the input")
    return out


def quant_matvec(w: np.ndarray, ggml_type: int, x: np.ndarray, n_out: int, w_size=None):
    w = np.ascontiguousarray(w, np.uint8) if ggml_type != 0 else np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(n_out, np.float32)
    rc = lib().fwc_quant_matvec(w.ctypes.data, w.nbytes if w_size is None else w_size, ggml_type, _f(x),
                                _f(y), x.size, n_out)
    return rc, y


def rms_norm(x, w, eps) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().fwc_rms_norm(_f(x), None if w is None else _f(np.ascontiguousarray(w, np.float32)), _f(out),
                       x.size, eps)
    return out


def rope_apply(qk, pos, n_heads, head_dim, cos, sin, neox=0) -> np.ndarray:
    qk = np.array(qk, np.float32, copy=True)
    lib().fwc_rope_apply(_f(qk), pos, n_heads, head_dim, _f(cos), _f(sin), neox)
    return qk


def softmax(x) -> np.ndarray:
    x = np.array(x, np.float32, copy=True)
    lib().fwc_softmax(_f(x), x.size)
    return x


def silu(x) -> np.ndarray:
    x = np.array(x, np.float32, copy=True)
    lib().fwc_silu(_f(x), x.size)
    return x


def gelu(x) -> np.ndarray:
    x = np.array(x, np.float32, copy=True)
    lib().fwc_gelu(_f(x), x.size)
    return x


def gelu_fast(x) -> np.ndarray:
    x = np.array(x, np.float32, copy=True)
    lib().fwc_gelu_fast(_f(x), x.size)
    return x


def argmax(x) -> int:
    x = np.ascontiguousarray(x, np.float32)
    return int(lib().fwc_argmax(_f(x), x.size))


def attention_core(q, kc, vc, n_head, n_kv, head_dim, pos) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    kc = np.ascontiguousarray(kc, np.float32)
    vc = np.ascontiguousarray(vc, np.float32)
    out = np.zeros(n_head * head_dim, np.float32)
    scores = np.zeros(n_head * (pos + 1), np.float32)
    lib().fwc_attention_core(_f(q), _f(kc), _f(vc), _f(out), n_head, n_kv, head_dim, pos, _f(scores))
    return out


class OracleModel:
    """transformer_t + transformer_forward on the CPU restatement."""

    def __init__(self, host: "fwgpu.HostModel"):
        self.host = host
        self.m = lib().fwc_model_init(host.data, host.data_size, host.tensors, host.n_tensors,
                                      C.byref(host.cfg), host.n_ctx, _f(host.cos), _f(host.sin))
        if not self.m:
            raise ValueError("fwc_model_init failed")
        self.n_vocab = host.cfg.n_vocab

    def forward(self, token: int, pos: int) -> np.ndarray:
        p = lib().fwc_forward(self.m, token, pos)
        if not p:
            raise ValueError("fwc_forward returned NULL")
        return np.ctypeslib.as_array(p, shape=(self.n_vocab,)).copy()

    def forward_raw(self, token: int, pos: int):
        return lib().fwc_forward(self.m, token, pos)

    def trace(self) -> np.ndarray:
        c = self.host.cfg
        p = lib().fwc_trace(self.m)
        return np.ctypeslib.as_array(p, shape=(2 * c.n_layer, c.n_embd)).copy()

    def kv(self, layer: int, pos: int):
        kvd = self.host.cfg.n_head_kv * self.host.cfg.head_dim
        if not (0 <= layer < self.host.cfg.n_layer and 0 <= pos < self.host.n_ctx):
            raise ValueError("kv: row outside the cache")
        k = np.ctypeslib.as_array(lib().fwc_kv_k(self.m, layer, pos), shape=(kvd,)).copy()
        v = np.ctypeslib.as_array(lib().fwc_kv_v(self.m, layer, pos), shape=(kvd,)).copy()
        return k, v

    def set_kv(self, layer: int, pos0: int, k: np.ndarray, v: np.ndarray):
        kvd = self.host.cfg.n_head_kv * self.host.cfg.head_dim
        if not 0 <= layer < self.host.cfg.n_layer or pos0 < 0 or pos0 + k.shape[0] > self.host.n_ctx or \
                k.shape != v.shape or k.shape[1:] != (kvd,):
            raise ValueError("set_kv: rows outside the cache or of the wrong width")
        for i in range(k.shape[0]):
            np.ctypeslib.as_array(lib().fwc_kv_k(self.m, layer, pos0 + i), shape=(kvd,))[:] = k[i]
            np.ctypeslib.as_array(lib().fwc_kv_v(self.m, layer, pos0 + i), shape=(kvd,))[:] = v[i]

    def generate_greedy(self, prompt, n_gen: int) -> np.ndarray:
        pr = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(n_gen, np.uint32)
        if lib().fwc_generate_greedy(self.m, pr.ctypes.data_as(u32p), pr.size, n_gen,
                                     out.ctypes.data_as(u32p)) != 0:
            raise ValueError("fwc_generate_greedy failed")
        return out

    def generate_sampled(self, prompt, n_gen: int, temperature: float, top_p: float, penalty: float,
                         seed: int) -> np.ndarray:
        pr = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(n_gen, np.uint32)
        if lib().fwc_generate_sampled(self.m, pr.ctypes.data_as(u32p), pr.size, n_gen, temperature, top_p,
                                      penalty, seed, out.ctypes.data_as(u32p)) != 0:
            raise ValueError("fwc_generate_sampled failed")
        return out

    def close(self):
        if getattr(self, "m", None):
            lib().fwc_model_free(self.m)
            self.m = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


def sample(logits, hist, temperature, top_p, penalty, rng_state: int):
    """One sampling decision; returns (token, new xorshift64 state)."""
    lg = np.ascontiguousarray(logits, np.float32)
    h = np.ascontiguousarray(hist, np.uint32)
    st = C.c_uint64(rng_state)
    t = lib().fwc_sample(_f(lg), lg.size, h.ctypes.data_as(u32p), h.size, temperature, top_p, penalty,
                         C.byref(st))
    return int(t), int(st.value)
