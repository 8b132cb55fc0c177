"""The C-ABI libraries load and export every entry point include/*.h declares;
argument validation follows the reference's conventions.  No GPU needed: only
calls that are rejected before any device work are made here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import fwgpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header, prefix):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    names = set(re.findall(r"\b(" + prefix + r"\w+)\s*\(", text))
    return sorted(names)


def test_gpu_library_exports_every_declared_symbol():
    names = declared("forword_gpu.h", "forword_gpu_")
    assert len(names) >= 25
    lib = C.CDLL(fwgpu.GPU_LIB)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_host_library_exports_every_declared_symbol():
    names = declared("fw_host.h", "fwh_")
    assert len(names) >= 25
    lib = C.CDLL(fwgpu.HOST_LIB)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_init_rejects_invalid_arguments():
    L = fwgpu.gpu_lib()
    h = C.c_void_p()
    cfg = fwgpu.Config()
    assert L.forword_gpu_init(C.byref(h), None, 0, None, 0, C.byref(cfg), 0, None, None) == -1
    assert not h.value
    assert "invalid" in fwgpu.last_error()
    assert L.forword_gpu_init(None, None, 0, None, 0, None, 0, None, None) == -1


def test_model_calls_reject_null_handle():
    L = fwgpu.gpu_lib()
    assert not L.forword_gpu_forward(None, 0, 0)
    nxt = C.c_uint32()
    assert L.forword_gpu_forward_argmax(None, 0, 0, C.byref(nxt)) == -1
    assert L.forword_gpu_kv_write(None, 0, 0, 1, None, None) == -1
    assert L.forword_gpu_layer_trace(None, None) == -1
    assert L.forword_gpu_n_ctx(None) == 0
    assert L.forword_gpu_status(None) == -1
    L.forword_gpu_free(None)


def test_init_rejects_unsupported_variant():
    """An unknown norm type is refused with -1, not run."""
    sp = fwgpu.spec(256, 512, 2, 8, 2, 1000, 64)
    with fwgpu.HostModel(synth=sp) as host:
        cfg = fwgpu.Config.from_buffer_copy(host.cfg)
        cfg.norm_type = 5
        h = C.c_void_p()
        rc = fwgpu.gpu_lib().forword_gpu_init(C.byref(h), host.data, host.data_size, host.tensors,
                                              host.n_tensors, C.byref(cfg), host.n_ctx,
                                              host.cos.ctypes.data_as(fwgpu.fp), host.sin.ctypes.data_as(fwgpu.fp))
        assert rc == -1 and not h.value
        assert "unknown norm or RoPE type" in fwgpu.last_error()


def test_operator_argument_checks_match_reference():
    """quant_matvec.c:274-289 conditions return -1 before any launch."""
    L = fwgpu.gpu_lib()
    w = C.c_void_p(16)   # never dereferenced: every call below fails validation first
    x = C.c_void_p(32)
    y = C.c_void_p(48)
    assert L.forword_gpu_quant_matvec(None, 34, 8, x, y, 32, 1, None) == -1
    assert L.forword_gpu_quant_matvec(w, 34, 8, x, y, 0, 1, None) == -1
    assert L.forword_gpu_quant_matvec(w, 34, 8, x, y, 32, 0, None) == -1
    assert L.forword_gpu_quant_matvec(w, 34, 3, x, y, 32, 1, None) == -1       # Q4_1: unsupported
    assert L.forword_gpu_quant_matvec(w, 34, 8, x, y, 40, 1, None) == -1       # in % 32
    assert L.forword_gpu_quant_matvec(w, 33, 8, x, y, 32, 1, None) == -1       # too small
    assert L.forword_gpu_dequant(w, 35, 8, y, 32, None) == -1
    assert L.forword_gpu_dequant(w, 34, 8, y, 64, None) == -1
    assert L.forword_gpu_tensor_rms_norm(w, w, y, 4, 0.0, None) == -1          # tensor_ops.c:46-48
    assert L.forword_gpu_tensor_rms_norm(w, w, y, 4, float("nan"), None) == -1
    assert L.forword_gpu_tensor_silu(None, y, 4, None) == -1
    assert L.forword_gpu_tensor_add(w, None, y, 4, None) == -1
    assert L.forword_gpu_tensor_matvec_f32(w, x, y, 0, 5, None) == -1
    assert L.forword_gpu_attention(w, w, w, y, 6, 4, 48, 10, 0, None) == -1    # n_head % n_kv
    assert L.forword_gpu_attention(w, w, w, y, 6, 6, 48, 10, 10, None) == -1   # pos >= n_ctx
    assert L.forword_gpu_rope_apply(y, 0, 1, 47, w, w, 0, None) == -1          # odd head_dim
    assert L.forword_gpu_get_row(w, 34, 8, 32, 1, y, None) == -1               # row outside tensor


@pytest.mark.parametrize("n", [0, 1])
def test_synth_rejects_bad_spec(n):
    sp = fwgpu.spec(250 + n, 512, 2, 8, 2, 1000, 64)     # n_embd not a multiple of 32
    assert fwgpu.host_lib().fwh_synth_size(C.byref(sp)) == 0
    with pytest.raises(ValueError):
        fwgpu.HostModel(synth=sp)


def test_header_struct_layouts():
    """ctypes mirrors of the ABI structs have the C layout (natural alignment)."""
    assert C.sizeof(fwgpu.TensorDesc) == 8 + 4 + 4 + 32 + 4 + 4 + 8 + 8
    assert C.sizeof(fwgpu.Config) == 4 * 21
    assert np.dtype(np.uint64).itemsize == 8


def test_qwen2_synth_config():
    """A qwen2 file gets the architecture's block settings (model_config.c:161-168):
    q/k/v biases on, RoPE base raised to 1e6; the writer emits one F32 bias per
    q/k/v projection."""
    sp = fwgpu.spec(256, 512, 2, 8, 2, 1000, 64, 10000.0, arch="qwen2")
    with fwgpu.HostModel(synth=sp) as host:
        c = host.cfg
        assert c.arch == 3 and c.use_qkv_bias == 1 and c.rope_freq_base == 1e6
        names = {host.tensors[i].name.decode(): host.tensors[i] for i in range(host.n_tensors)}
        for l in range(2):
            for r, n in (("q", 256), ("k", 64), ("v", 64)):
                t = names[f"blk.{l}.attn_{r}.bias"]
                assert t.ggml_type == 0 and t.n_dims == 1 and t.dims[0] == n



@pytest.mark.parametrize("arch,expect", [
    # (arch, norm, act, gate, rope, qkv_bias, parallel, embd_scale) as model_config.c:148-217 sets them
    ("llama", (2, 0, 0, 1, 0, 0, 0, 1.0)),
    ("gemma", (5, 0, 2, 1, 0, 0, 0, 16.0)),
    ("phi2", (6, 1, 2, 0, 1, 0, 1, 1.0)),
    ("gpt2", (1, 1, 1, 0, 2, 1, 0, 1.0)),
])
def test_synth_arch_config(arch, expect):
    """Each synthetic architecture reads back with the reference's per-architecture
    block settings (the config reader mirrors model_config.c)."""
    sp = fwgpu.spec(256, 512, 1, 4, 4, 300, 32, 10000.0, arch=arch)
    with fwgpu.HostModel(synth=sp) as host:
        c = host.cfg
        got = (c.arch, c.norm_type, c.act_type, c.use_ffn_gate, c.rope_type, c.use_qkv_bias, c.parallel_res,
               round(c.embd_scale, 4))
        assert got == expect
        names = {host.tensors[i].name.decode() for i in range(host.n_tensors)}
        assert ("output.weight" in names) == (arch in ("llama", "phi2"))        # gemma, gpt2: tied head
        assert ("blk.0.attn_qkv.weight" in names) == (arch == "gpt2")
        assert ("position_embd.weight" in names) == (arch == "gpt2")
        assert ("blk.0.ffn_gate.weight" in names) == (arch in ("llama", "gemma"))
