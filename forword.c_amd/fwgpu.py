"""ctypes binding of the forword MI355X decode path.

Mirrors the reference's interfaces for the per-token forward:

* ``HostModel``   - what transformer_init does on the host (transformer.c:14-128):
                    open/parse the GGUF (gguf.c:256-353), read the config
                    (model_config.c:61-220), resolve max_ctx (transformer.c:43-52)
                    and build the RoPE tables (rope.c:6-17).
* ``GpuModel``    - transformer_forward (transformer.c:149-326) and the CLI's
                    prefill/greedy loop (main.c:145-217) on the GPU through the
                    forword_gpu_* C ABI (include/forword_gpu.h).
* ``ops``         - operator-level entry points on device pointers
                    (quant_matvec, rms_norm, rope_apply, attention, silu, argmax, ...).

The GPU library is required: every GPU call raises if lib/libforword_gpu.so is
missing or fails to load; nothing falls back to a CPU path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBDIR = os.path.join(HERE, "lib")
HOST_LIB = os.environ.get("FW_HOST_LIB") or os.path.join(LIBDIR, "libfw_host.so")   # override: instrumented builds
GPU_LIB = os.environ.get("FW_GPU_LIB") or os.path.join(LIBDIR, "libforword_gpu.so")   # override: A/B builds

GGML_F32, GGML_Q4_0, GGML_Q5_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 2, 6, 8, 12, 14
BLOCK_BYTES = {GGML_Q4_0: 18, GGML_Q5_0: 22, GGML_Q8_0: 34, GGML_Q4_K: 144, GGML_Q6_K: 210}
BLOCK_VALUES = {GGML_Q4_0: 32, GGML_Q5_0: 32, GGML_Q8_0: 32, GGML_Q4_K: 256, GGML_Q6_K: 256}
# Architectures the synthetic writer emits, as FORWORD_ARCH_* values (model_config.h:12-24).
SYNTH_ARCHS = {"gpt2": 1, "llama": 2, "qwen2": 3, "gemma": 5, "phi2": 6}
TYPE_NAMES = {GGML_F32: "F32", GGML_Q4_0: "Q4_0", GGML_Q5_0: "Q5_0", GGML_Q8_0: "Q8_0", GGML_Q4_K: "Q4_K",
              GGML_Q6_K: "Q6_K"}

u32, u64, i32, f32 = C.c_uint32, C.c_uint64, C.c_int32, C.c_float
vp, sz = C.c_void_p, C.c_size_t
fp = C.POINTER(C.c_float)
u32p = C.POINTER(C.c_uint32)


class TensorDesc(C.Structure):
    """forword_gpu_tensor_t (fields of gguf_tensor_t, gguf.h:16-24)."""
    _fields_ = [("name", C.c_char_p), ("n_dims", u32), ("dims", u64 * 4), ("ggml_type", u32),
                ("offset", u64), ("byte_size", u64)]


class Config(C.Structure):
    """forword_gpu_config_t (fields of model_config_t, model_config.h:47-89)."""
    _fields_ = [("arch", u32), ("n_vocab", u32), ("n_ctx", u32), ("n_embd", u32), ("n_layer", u32),
                ("n_head", u32), ("n_head_kv", u32), ("n_ff", u32), ("head_dim", u32), ("n_rot", u32),
                ("norm_type", u32), ("act_type", u32), ("rope_type", u32),
                ("use_ffn_gate", i32), ("use_qkv_bias", i32), ("use_alibi", i32), ("parallel_res", i32),
                ("norm_eps", f32), ("rope_freq_base", f32), ("rope_freq_scale", f32), ("embd_scale", f32)]


class SynthSpec(C.Structure):
    """fwh_synth_spec_t: a seeded random-init llama-shaped model."""
    _fields_ = [("n_embd", u32), ("n_ff", u32), ("n_layer", u32), ("n_head", u32), ("n_head_kv", u32),
                ("n_vocab", u32), ("n_ctx", u32), ("rope_freq_base", f32), ("norm_eps", f32),
                ("linear_type", u32), ("embd_type", u32), ("output_type", u32), ("seed", u64),
                ("w_std", f32), ("norm_std", f32), ("threads", u32), ("arch", u32), ("mix_type", u32)]


def spec(n_embd, n_ff, n_layer, n_head, n_head_kv, n_vocab, n_ctx, rope_freq_base=10000.0,
         norm_eps=1e-5, linear_type=GGML_Q8_0, embd_type=GGML_Q8_0, output_type=GGML_Q8_0,
         seed=1, w_std=0.02, norm_std=0.01, threads=0, arch="llama", mix_type=0) -> SynthSpec:
    """Synthetic model shape.  arch "qwen2" adds attn_{q,k,v}.bias per layer; "gemma"
    (gated GELU-tanh FFN, embedding times sqrt(n_embd)) ties the lm-head to token_embd;
    "phi2" is the LayerNorm / parallel-residual / plain-FFN / NEOX-RoPE block with norm
    and output-projection biases.  mix_type != 0 gives attn_v and ffn_down of the even
    layers that type instead of linear_type."""
    return SynthSpec(n_embd, n_ff, n_layer, n_head, n_head_kv, n_vocab, n_ctx, rope_freq_base,
                     norm_eps, linear_type, embd_type, output_type, seed, w_std, norm_std, threads,
                     SYNTH_ARCHS[arch], mix_type)


# Workload shapes (dims, heads, ffn, vocab, RoPE base) of the configurations this path is measured on.
def spec_tiny(seed=20240601, **kw):
    """dim 288, ffn 768, 6 layers, 6/6 heads (hd 48), vocab 32000, ctx 256, all Q8_0, theta 1e4."""
    return spec(288, 768, 6, 6, 6, 32000, 256, 10000.0, seed=seed, **kw)


def spec_8b(seed=8, n_ctx=768, **kw):
    """Llama-3-8B shape: dim 4096, 32 layers, 32/8 heads, ffn 14336, vocab 128256, theta 5e5,
    Q4_0 linears, Q8_0 embedding and output."""
    kw.setdefault("linear_type", GGML_Q4_0)
    return spec(4096, 14336, 32, 32, 8, 128256, n_ctx, 500000.0, seed=seed, **kw)


def spec_70b(seed=70, n_ctx=384, **kw):
    """Llama-3-70B shape: dim 8192, 80 layers, 64/8 heads, ffn 28672, vocab 128256, theta 5e5."""
    kw.setdefault("linear_type", GGML_Q4_0)
    return spec(8192, 28672, 80, 64, 8, 128256, n_ctx, 500000.0, seed=seed, **kw)


def spec_qwen2_7b(seed=27, n_ctx=768, **kw):
    """Qwen2-7B shape: dim 3584, 28 layers, 28/4 heads (hd 128, group 7), ffn 18944, vocab
    152064, q/k/v biases, RoPE base 1e6 (set by the config loader); Q4_0 linears."""
    kw.setdefault("linear_type", GGML_Q4_0)
    return spec(3584, 18944, 28, 28, 4, 152064, n_ctx, 1000000.0, seed=seed, arch="qwen2", **kw)


def spec_phi2(seed=22, n_ctx=768, **kw):
    """Phi-2 shape: dim 2560, 32 layers, 32/32 heads (hd 80), ffn 10240, vocab 51200, LayerNorm,
    parallel residual, plain GELU FFN, NEOX RoPE; Q4_0 linears."""
    kw.setdefault("linear_type", GGML_Q4_0)
    return spec(2560, 10240, 32, 32, 32, 51200, n_ctx, 10000.0, seed=seed, arch="phi2", **kw)


def spec_gpt2_xl(seed=48, n_ctx=768, **kw):
    """GPT-2 XL shape: dim 1600, 48 layers, 25 heads (hd 64), ffn 6400, vocab 50257, learned
    positions, fused attn_qkv, LayerNorm, erf-GELU FFN with biases; Q8_0 linears."""
    kw.setdefault("linear_type", GGML_Q8_0)
    return spec(1600, 6400, 48, 25, 25, 50257, n_ctx, 10000.0, seed=seed, arch="gpt2", **kw)


_host = None
_gpu = None


def _sig(lib, name, res, args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = args
    return fn


def host_lib():
    global _host
    if _host is None:
        if not os.path.exists(HOST_LIB):
            raise RuntimeError(f"{HOST_LIB} is not built (run __graft_entry__.build())")
        L = C.CDLL(HOST_LIB)
        _sig(L, "fwh_gguf_open", vp, [C.c_char_p, C.c_char_p, sz])
        _sig(L, "fwh_gguf_open_memory", vp, [vp, sz, C.c_char_p, sz])
        _sig(L, "fwh_gguf_close", None, [vp])
        _sig(L, "fwh_gguf_version", u32, [vp])
        _sig(L, "fwh_gguf_alignment", u32, [vp])
        _sig(L, "fwh_gguf_data_offset", u64, [vp])
        _sig(L, "fwh_gguf_data", vp, [vp, C.POINTER(sz)])
        _sig(L, "fwh_gguf_n_tensors", sz, [vp])
        _sig(L, "fwh_gguf_tensors", C.POINTER(TensorDesc), [vp])
        _sig(L, "fwh_gguf_find_tensor", C.c_long, [vp, C.c_char_p])
        _sig(L, "fwh_gguf_kv_type", C.c_int, [vp, C.c_char_p])
        _sig(L, "fwh_gguf_get_u32", C.c_int, [vp, C.c_char_p, u32p])
        _sig(L, "fwh_gguf_get_f32", C.c_int, [vp, C.c_char_p, fp])
        _sig(L, "fwh_gguf_get_str", C.c_int, [vp, C.c_char_p, C.c_char_p, sz])
        _sig(L, "fwh_gguf_array_len", C.c_int64, [vp, C.c_char_p])
        _sig(L, "fwh_config", C.c_int, [vp, C.POINTER(Config)])
        _sig(L, "fwh_resolve_ctx", sz, [C.POINTER(Config), sz])
        _sig(L, "fwh_rope_tables", None, [fp, fp, sz, sz, f32])
        _sig(L, "fwh_f32_to_f16", C.c_uint16, [f32])
        _sig(L, "fwh_f16_to_f32", f32, [C.c_uint16])
        _sig(L, "fwh_randn", None, [u64, f32, fp, sz])
        _sig(L, "fwh_block_bytes", sz, [u32])
        _sig(L, "fwh_quantize", sz, [u32, fp, sz, vp])
        _sig(L, "fwh_synth_size", sz, [C.POINTER(SynthSpec)])
        _sig(L, "fwh_synth_write", sz, [C.POINTER(SynthSpec), vp, sz])
        _sig(L, "fwh_synth_write_file", C.c_int, [C.POINTER(SynthSpec), C.c_char_p])
        _sig(L, "fwh_synth_alloc", vp, [C.POINTER(SynthSpec), C.POINTER(sz)])
        _sig(L, "fwh_synth_release", None, [vp, sz])
        _sig(L, "fwh_synth_matrix", sz, [u32, sz, sz, u64, f32, u32, vp, u32])
        _sig(L, "fwh_default_threads", u32, [])
        _host = L
    return _host


def gpu_lib():
    """Load lib/libforword_gpu.so (or the build named by FORWORD_GPU_LIB, for A/B
    comparisons of kernel variants); raises when it is missing (no CPU fallback exists)."""
    global _gpu
    if _gpu is None:
        path = os.environ.get("FORWORD_GPU_LIB", GPU_LIB)
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built (run __graft_entry__.build())")
        L = C.CDLL(path)
        _sig(L, "forword_gpu_init", C.c_int, [C.POINTER(vp), vp, sz, C.POINTER(TensorDesc), sz,
                                               C.POINTER(Config), sz, fp, fp])
        _sig(L, "forword_gpu_free", None, [vp])
        _sig(L, "forword_gpu_forward", fp, [vp, u32, sz])
        _sig(L, "forword_gpu_forward_argmax", C.c_int, [vp, u32, sz, u32p])
        _sig(L, "forword_gpu_generate_greedy", C.c_int, [vp, u32p, sz, sz, u32p])
        _sig(L, "forword_gpu_decode", C.c_int, [vp, sz, u32p])
        _sig(L, "forword_gpu_decode_from", C.c_int, [vp, u32, sz, sz, u32p])
        _sig(L, "forword_gpu_prefill", fp, [vp, u32p, sz, sz])
        _sig(L, "forword_gpu_generate", C.c_int, [vp, u32p, sz, sz, f32, f32, f32, u64, u32p])
        _sig(L, "forword_gpu_prefill_argmax", C.c_int, [vp, u32p, sz, sz, u32p])
        _sig(L, "forword_gpu_ffn_swiglu", C.c_int, [vp, vp, sz, u32, vp, vp, sz, sz, vp])
        _sig(L, "forword_gpu_kv_write", C.c_int, [vp, sz, sz, sz, fp, fp])
        _sig(L, "forword_gpu_kv_read", C.c_int, [vp, sz, sz, sz, fp, fp])
        _sig(L, "forword_gpu_layer_trace", C.c_int, [vp, fp])
        _sig(L, "forword_gpu_n_ctx", sz, [vp])
        _sig(L, "forword_gpu_stream", vp, [vp])
        _sig(L, "forword_gpu_step_impl", C.c_int, [vp])
        _sig(L, "forword_gpu_status", C.c_int, [vp])
        _sig(L, "forword_gpu_phase_times", C.c_int, [vp, C.POINTER(C.c_double), sz])
        _sig(L, "forword_gpu_last_error", C.c_char_p, [])
        _sig(L, "forword_gpu_quant_matvec", C.c_int, [vp, sz, u32, vp, vp, sz, sz, vp])
        _sig(L, "forword_gpu_dequant", C.c_int, [vp, sz, u32, vp, sz, vp])
        _sig(L, "forword_gpu_get_row", C.c_int, [vp, sz, u32, sz, sz, vp, vp])
        _sig(L, "forword_gpu_rms_norm", C.c_int, [vp, vp, vp, sz, f32, vp])
        _sig(L, "forword_gpu_rope_apply", C.c_int, [vp, sz, sz, sz, vp, vp, C.c_int, vp])
        _sig(L, "forword_gpu_attention", C.c_int, [vp, vp, vp, vp, sz, sz, sz, sz, sz, vp])
        _sig(L, "forword_gpu_silu_mul", C.c_int, [vp, vp, vp, sz, vp])
        _sig(L, "forword_gpu_tensor_matvec_f32", C.c_int, [vp, vp, vp, sz, sz, vp])
        _sig(L, "forword_gpu_tensor_add", C.c_int, [vp, vp, vp, sz, vp])
        _sig(L, "forword_gpu_tensor_rms_norm", C.c_int, [vp, vp, vp, sz, f32, vp])
        _sig(L, "forword_gpu_tensor_silu", C.c_int, [vp, vp, sz, vp])
        _sig(L, "forword_gpu_argmax", C.c_int, [vp, sz, vp, vp])
        _sig(L, "forword_gpu_dev_alloc", vp, [sz])
        _sig(L, "forword_gpu_dev_free", C.c_int, [vp])
        _sig(L, "forword_gpu_memcpy_h2d", C.c_int, [vp, vp, sz])
        _sig(L, "forword_gpu_memcpy_d2h", C.c_int, [vp, vp, sz])
        _sig(L, "forword_gpu_memset", C.c_int, [vp, C.c_int, sz])
        _sig(L, "forword_gpu_synchronize", C.c_int, [vp])
        _gpu = L
    return _gpu


def last_error() -> str:
    return (gpu_lib().forword_gpu_last_error() or b"").decode()


class ForwordError(RuntimeError):
    pass


def _check(rc, what):
    if rc != 0:
        raise ForwordError(f"{what} failed: {last_error()}")


# ── host side ─────────────────────────────────────────────────────────────────

def f32_to_f16(x: float) -> int:
    return host_lib().fwh_f32_to_f16(x)


def randn(seed: int, n: int, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    host_lib().fwh_randn(seed, std, out.ctypes.data_as(fp), n)
    return out


def synth_matrix(ggml_type: int, rows: int, cols: int, seed: int, scale_std: float = 0.02,
                 subnormal_every: int = 0, threads: int = 0) -> np.ndarray:
    """Microbenchmark matrix of GGUF blocks (codes uniform, scales fp16(|N(0,1)|*scale_std))."""
    n = rows * (cols // BLOCK_VALUES[ggml_type]) * BLOCK_BYTES[ggml_type]
    out = np.empty(n, np.uint8)
    got = host_lib().fwh_synth_matrix(ggml_type, rows, cols, seed, scale_std, subnormal_every,
                                      out.ctypes.data, threads)
    if got != n:
        raise ValueError("fwh_synth_matrix failed")
    return out


def quantize(ggml_type: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size // BLOCK_VALUES[ggml_type] * BLOCK_BYTES[ggml_type], np.uint8)
    if host_lib().fwh_quantize(ggml_type, x.ctypes.data_as(fp), x.size, out.ctypes.data) != out.size:
        raise ValueError("fwh_quantize failed")
    return out


class HostModel:
    """A GGUF model as transformer_init sees it on the host."""

    def __init__(self, *, path: str | None = None, synth: SynthSpec | None = None,
                 image: bytes | None = None, max_ctx: int = 0):
        H = host_lib()
        err = C.create_string_buffer(256)
        self._synth = None
        self._image = None
        if synth is not None:
            n = sz(0)
            p = H.fwh_synth_alloc(C.byref(synth), C.byref(n))
            if not p:
                raise ValueError("synthetic model generation failed (bad spec or out of memory)")
            self._synth = (p, n.value)
            self.g = H.fwh_gguf_open_memory(p, n.value, err, 256)
        elif image is not None:
            self._image = C.create_string_buffer(bytes(image), len(image))
            self.g = H.fwh_gguf_open_memory(C.addressof(self._image), len(image), err, 256)
        else:
            self.g = H.fwh_gguf_open(path.encode(), err, 256)
        if not self.g:
            self.close()
            raise ValueError(f"gguf open failed: {err.value.decode()}")
        self.cfg = Config()
        if H.fwh_config(self.g, C.byref(self.cfg)) != 0:
            self.close()
            raise ValueError("model config load failed")
        self.n_ctx = H.fwh_resolve_ctx(C.byref(self.cfg), max_ctx)
        if not self.n_ctx:
            self.close()
            raise ValueError("invalid context length")
        half = self.cfg.head_dim // 2
        self.cos = np.zeros(max(self.n_ctx * half, 1), np.float32)
        self.sin = np.zeros(max(self.n_ctx * half, 1), np.float32)
        if self.cfg.rope_type != 2 and half:
            H.fwh_rope_tables(self.cos.ctypes.data_as(fp), self.sin.ctypes.data_as(fp), self.n_ctx,
                              self.cfg.head_dim, self.cfg.rope_freq_base)
        dsz = sz(0)
        self.data = H.fwh_gguf_data(self.g, C.byref(dsz))
        self.data_size = dsz.value
        self.n_tensors = H.fwh_gguf_n_tensors(self.g)
        self.tensors = H.fwh_gguf_tensors(self.g)

    def tensor(self, name: str) -> TensorDesc:
        i = host_lib().fwh_gguf_find_tensor(self.g, name.encode())
        if i < 0:
            raise KeyError(name)
        return self.tensors[i]

    def tensor_bytes(self, name: str) -> np.ndarray:
        t = self.tensor(name)
        return np.ctypeslib.as_array((C.c_uint8 * t.byte_size).from_address(self.data + t.offset)).copy()

    def close(self):
        H = host_lib()
        if getattr(self, "g", None):
            H.fwh_gguf_close(self.g)
            self.g = None
        if self._synth:
            H.fwh_synth_release(*self._synth)
            self._synth = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


# ── GPU model ─────────────────────────────────────────────────────────────────

class GpuModel:
    """transformer_forward on the GPU (forword_gpu_init/forward/... in include/forword_gpu.h)."""

    def __init__(self, host: HostModel):
        L = gpu_lib()
        self.host = host
        h = vp()
        _check(L.forword_gpu_init(C.byref(h), host.data, host.data_size, host.tensors, host.n_tensors,
                                  C.byref(host.cfg), host.n_ctx, host.cos.ctypes.data_as(fp),
                                  host.sin.ctypes.data_as(fp)), "forword_gpu_init")
        self.h = h
        self.n_vocab = host.cfg.n_vocab

    @property
    def stream(self):
        return gpu_lib().forword_gpu_stream(self.h)

    def phase_times(self) -> np.ndarray:
        """Mean per-phase microseconds of the last persistent launch (needs
        FORWORD_GPU_PHASE_TIMES=1 at construction)."""
        n = 5 * self.host.cfg.n_layer + 1
        out = np.zeros(n, np.float64)
        got = gpu_lib().forword_gpu_phase_times(self.h, out.ctypes.data_as(C.POINTER(C.c_double)), n)
        if got < 0:
            raise ForwordError(f"phase_times failed: {last_error()}")
        return out[:got]

    def status(self):
        """Wait for the queued work; raise if a persistent launch gave up at a bounded wait."""
        _check(gpu_lib().forword_gpu_status(self.h), "status")

    @property
    def persistent(self) -> bool:
        """True when whole token steps run as one persistent kernel."""
        return gpu_lib().forword_gpu_step_impl(self.h) == 1

    def forward(self, token: int, pos: int) -> np.ndarray:
        p = gpu_lib().forword_gpu_forward(self.h, token, pos)
        if not p:
            raise ForwordError(f"forword_gpu_forward failed: {last_error()}")
        return np.ctypeslib.as_array(p, shape=(self.n_vocab,)).copy()

    def forward_raw(self, token: int, pos: int):
        """The raw pointer result (None on error), as transformer_forward returns it."""
        return gpu_lib().forword_gpu_forward(self.h, token, pos)

    def forward_argmax(self, token: int, pos: int) -> int:
        nxt = u32(0)
        _check(gpu_lib().forword_gpu_forward_argmax(self.h, token, pos, C.byref(nxt)), "forward_argmax")
        return nxt.value

    def prefill(self, tokens, pos0: int = 0) -> np.ndarray:
        """Batched forward of tokens at positions pos0..; logits of the last one."""
        tk = np.ascontiguousarray(tokens, np.uint32)
        p = gpu_lib().forword_gpu_prefill(self.h, tk.ctypes.data_as(u32p), tk.size, pos0)
        if not p:
            raise ForwordError(f"forword_gpu_prefill failed: {last_error()}")
        return np.ctypeslib.as_array(p, shape=(self.n_vocab,)).copy()

    def prefill_argmax(self, tokens, pos0: int = 0) -> int:
        tk = np.ascontiguousarray(tokens, np.uint32)
        nxt = u32(0)
        _check(gpu_lib().forword_gpu_prefill_argmax(self.h, tk.ctypes.data_as(u32p), tk.size, pos0, C.byref(nxt)),
               "prefill_argmax")
        return nxt.value

    def generate(self, prompt, n_gen: int, temperature: float = 0.8, top_p: float = 0.9,
                 repetition_penalty: float = 1.1, seed: int = 12345) -> np.ndarray:
        """The CLI's sampled generation loop (main.c:145-217, sampler.c) on the device."""
        pr = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(n_gen, np.uint32)
        _check(gpu_lib().forword_gpu_generate(self.h, pr.ctypes.data_as(u32p), pr.size, n_gen, temperature, top_p,
                                              repetition_penalty, seed, out.ctypes.data_as(u32p)), "generate")
        return out

    def generate_greedy_batched(self, prompt, n_gen: int) -> np.ndarray:
        """Greedy generation with the batched prefill: the prompt in one pass, then
        the device-resident loop from the first generated token."""
        first = self.prefill_argmax(prompt, 0)
        if n_gen <= 1:
            return np.array([first][:n_gen], np.uint32)
        rest = self.decode_from(first, len(prompt), n_gen - 1)
        return np.concatenate([[first], rest]).astype(np.uint32)

    def generate_greedy(self, prompt, n_gen: int) -> np.ndarray:
        pr = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(n_gen, np.uint32)
        _check(gpu_lib().forword_gpu_generate_greedy(self.h, pr.ctypes.data_as(u32p), pr.size, n_gen,
                                                     out.ctypes.data_as(u32p)), "generate_greedy")
        return out

    def decode(self, n_steps: int, copy_out: bool = True):
        """Continue the device-resident greedy loop; without copy_out only queue the steps."""
        out = np.zeros(n_steps, np.uint32) if copy_out else None
        _check(gpu_lib().forword_gpu_decode(self.h, n_steps, out.ctypes.data_as(u32p) if copy_out else None),
               "decode")
        return out

    def decode_from(self, token: int, pos: int, n_steps: int, copy_out: bool = True):
        """Greedy loop entered at (token, pos), e.g. after a kv_write prefill."""
        out = np.zeros(n_steps, np.uint32) if copy_out else None
        _check(gpu_lib().forword_gpu_decode_from(self.h, token, pos, n_steps,
                                                 out.ctypes.data_as(u32p) if copy_out else None), "decode_from")
        return out

    def kv_write(self, layer: int, pos0: int, k: np.ndarray | None, v: np.ndarray | None):
        k = None if k is None else np.ascontiguousarray(k, np.float32)
        v = None if v is None else np.ascontiguousarray(v, np.float32)
        n = (k if k is not None else v).shape[0]
        _check(gpu_lib().forword_gpu_kv_write(self.h, layer, pos0, n,
                                              None if k is None else k.ctypes.data_as(fp),
                                              None if v is None else v.ctypes.data_as(fp)), "kv_write")

    def kv_read(self, layer: int, pos0: int, n_pos: int):
        kvd = self.host.cfg.n_head_kv * self.host.cfg.head_dim
        k = np.zeros((n_pos, kvd), np.float32)
        v = np.zeros((n_pos, kvd), np.float32)
        _check(gpu_lib().forword_gpu_kv_read(self.h, layer, pos0, n_pos, k.ctypes.data_as(fp),
                                             v.ctypes.data_as(fp)), "kv_read")
        return k, v

    def layer_trace(self) -> np.ndarray:
        c = self.host.cfg
        out = np.zeros((2 * c.n_layer, c.n_embd), np.float32)
        _check(gpu_lib().forword_gpu_layer_trace(self.h, out.ctypes.data_as(fp)), "layer_trace")
        return out

    def close(self):
        if getattr(self, "h", None):
            gpu_lib().forword_gpu_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


# ── device buffers for the operator-level entry points ───────────────────────

class DeviceBuffer:
    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = gpu_lib().forword_gpu_dev_alloc(max(self.nbytes, 1))
        if not self.ptr:
            raise ForwordError(f"device allocation of {nbytes} bytes failed: {last_error()}")

    @classmethod
    def from_array(cls, a: np.ndarray):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            _check(gpu_lib().forword_gpu_memcpy_h2d(b.ptr, a.ctypes.data, a.nbytes), "memcpy_h2d")
        return b

    def to_array(self, dtype, count=None) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(count, dtype)
        if out.nbytes:
            _check(gpu_lib().forword_gpu_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes), "memcpy_d2h")
        return out

    def free(self):
        if self.ptr:
            gpu_lib().forword_gpu_dev_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class ops:
    """Operator-level calls; arguments are DeviceBuffers, results synchronised."""

    @staticmethod
    def _sync(rc, what):
        _check(rc, what)
        _check(gpu_lib().forword_gpu_synchronize(None), "synchronize")

    @staticmethod
    def quant_matvec(w: DeviceBuffer, ggml_type, x: DeviceBuffer, y: DeviceBuffer, n_in, n_out,
                     w_size=None):
        ops._sync(gpu_lib().forword_gpu_quant_matvec(w.ptr, w.nbytes if w_size is None else w_size,
                                                     ggml_type, x.ptr, y.ptr, n_in, n_out, None),
                  "quant_matvec")

    @staticmethod
    def dequant(blocks: DeviceBuffer, ggml_type, out: DeviceBuffer, count):
        ops._sync(gpu_lib().forword_gpu_dequant(blocks.ptr, blocks.nbytes, ggml_type, out.ptr, count, None),
                  "dequant")

    @staticmethod
    def get_row(w: DeviceBuffer, ggml_type, n_cols, row, out: DeviceBuffer):
        ops._sync(gpu_lib().forword_gpu_get_row(w.ptr, w.nbytes, ggml_type, n_cols, row, out.ptr, None),
                  "get_row")

    @staticmethod
    def rms_norm(x, w, out, n, eps):
        ops._sync(gpu_lib().forword_gpu_rms_norm(x.ptr, None if w is None else w.ptr, out.ptr, n, eps, None),
                  "rms_norm")

    @staticmethod
    def rope_apply(qk, pos, n_heads, head_dim, cos, sin, neox=0):
        ops._sync(gpu_lib().forword_gpu_rope_apply(qk.ptr, pos, n_heads, head_dim, cos.ptr, sin.ptr, neox,
                                                   None), "rope_apply")

    @staticmethod
    def attention(q, k, v, out, n_head, n_kv, head_dim, n_ctx, pos):
        ops._sync(gpu_lib().forword_gpu_attention(q.ptr, k.ptr, v.ptr, out.ptr, n_head, n_kv, head_dim,
                                                  n_ctx, pos, None), "attention")

    @staticmethod
    def silu_mul(gate, up, out, n):
        ops._sync(gpu_lib().forword_gpu_silu_mul(gate.ptr, up.ptr, out.ptr, n, None), "silu_mul")

    @staticmethod
    def ffn_swiglu(w_gate, w_up, ggml_type, x, h, n_in, n_ff, stream=None, sync=True):
        rc = gpu_lib().forword_gpu_ffn_swiglu(w_gate.ptr, w_up.ptr, min(w_gate.nbytes, w_up.nbytes), ggml_type,
                                              x.ptr, h.ptr, n_in, n_ff, stream)
        if sync:
            ops._sync(rc, "ffn_swiglu")
        else:
            _check(rc, "ffn_swiglu")

    @staticmethod
    def tensor_matvec_f32(w, x, y, rows, cols):
        ops._sync(gpu_lib().forword_gpu_tensor_matvec_f32(w.ptr, x.ptr, y.ptr, rows, cols, None),
                  "tensor_matvec_f32")

    @staticmethod
    def tensor_add(a, b, out, n):
        ops._sync(gpu_lib().forword_gpu_tensor_add(a.ptr, b.ptr, out.ptr, n, None), "tensor_add")

    @staticmethod
    def tensor_rms_norm(x, w, out, n, eps):
        ops._sync(gpu_lib().forword_gpu_tensor_rms_norm(x.ptr, w.ptr, out.ptr, n, eps, None),
                  "tensor_rms_norm")

    @staticmethod
    def tensor_silu(x, out, n):
        ops._sync(gpu_lib().forword_gpu_tensor_silu(x.ptr, out.ptr, n, None), "tensor_silu")

    @staticmethod
    def argmax(logits, n, out_idx):
        ops._sync(gpu_lib().forword_gpu_argmax(logits.ptr, n, out_idx.ptr, None), "argmax")
