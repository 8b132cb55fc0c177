"""forword_gpu_attention_noalloc (decode attention, attention.c:142-164, with its
split partials in a fixed per-device array instead of allocated scratch),
called through the C ABI: bit-identical to forword_gpu_attention on the same
inputs for two calls in a row, the second one smaller, and a call whose
partials do not fit the array refused before anything is launched."""
import ctypes as C

import numpy as np
import pytest

import fw_cpu
import fwgpu
from fwgpu import DeviceBuffer as DB

pytestmark = pytest.mark.gpu
SZ = C.c_size_t


def noalloc_fn():
    f = fwgpu.gpu_lib().forword_gpu_attention_noalloc
    f.restype = C.c_int
    f.argtypes = [C.c_void_p] * 4 + [SZ] * 5 + [C.c_void_p]
    return f


def run_both(n_head, n_kv, hd, pos, seed):
    n_ctx = pos + 5
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    k = rng.standard_normal(n_ctx * n_kv * hd).astype(np.float32)
    v = rng.standard_normal(n_ctx * n_kv * hd).astype(np.float32)
    dq, dk, dv = DB.from_array(q), DB.from_array(k), DB.from_array(v)
    a, b = DB(n_head * hd * 4), DB(n_head * hd * 4)
    fwgpu.ops.attention(dq, dk, dv, a, n_head, n_kv, hd, n_ctx, pos)
    rc = noalloc_fn()(dq.ptr, dk.ptr, dv.ptr, b.ptr, n_head, n_kv, hd, n_ctx, pos, None)
    assert rc == 0, fwgpu.last_error()
    assert fwgpu.gpu_lib().forword_gpu_synchronize(None) == 0
    got, exp = b.to_array(np.float32), a.to_array(np.float32)
    ref = fw_cpu.attention_core(q, k, v, n_head, n_kv, hd, pos)
    return got, exp, ref


def test_noalloc_attention_matches_allocating_entry_point():
    # 32 / 8 heads of 128 at position 3000: 128 splits, 2.1 MB of partials;
    # then a smaller call (8 / 2 heads of 64 at position 100) reusing the array
    for cfg, seed in (((32, 8, 128, 3000), 1), ((8, 2, 64, 100), 2)):
        got, exp, ref = run_both(*cfg, seed)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), cfg
        err = np.abs(got.astype(np.float64) - ref)
        assert np.all(err <= 2e-3 + 1e-3 * np.abs(ref)), (cfg, err.max())


def test_noalloc_attention_refuses_oversized_partials():
    # 64 heads of 256 at position 5000: 64 x 128 x 258 floats = 8.45 MB > 8 MiB
    buf = DB(4096)
    rc = noalloc_fn()(buf.ptr, buf.ptr, buf.ptr, buf.ptr, 64, 8, 256, 6000, 5000, None)
    assert rc == -1
    assert "scratch" in fwgpu.last_error()
    # the refusal leaves the entry point usable
    got, exp, _ = run_both(16, 8, 64, 40, 3)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
