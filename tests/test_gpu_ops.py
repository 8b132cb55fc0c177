"""Operator-level parity of the HIP kernels (through the C ABI) with the oracle
and the reference's golden vectors.  Integer/byte work (dequantisation,
argmax) must be bit-exact; floating-point reductions are held to the decode
path's tolerance (max-abs 2e-3 / rel 1e-3) and to a tighter error bound
relative to sum |w x|."""
import numpy as np
import pytest

import fw_cpu
import fwgpu
import golden_specs as gs
from fwgpu import DeviceBuffer as DB, ops

pytestmark = pytest.mark.gpu
Q4, Q5, Q8, F32 = fwgpu.GGML_Q4_0, fwgpu.GGML_Q5_0, fwgpu.GGML_Q8_0, fwgpu.GGML_F32
ATOL, RTOL = 2e-3, 1e-3      # decode-path tolerance on activations and logits


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bits_equal_nan_aware(got, exp):
    got, exp = np.asarray(got, np.float32), np.asarray(exp, np.float32)
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got[~nan]), bits(exp[~nan]))


def gpu_dequant(blocks, t):
    n = blocks.size // fwgpu.BLOCK_BYTES[t] * 32
    b, o = DB.from_array(blocks), DB(n * 4)
    ops.dequant(b, t, o, n)
    return o.to_array(np.float32)


def test_fp16_scale_conversion_all_65536():
    """Every fp16 bit pattern as a Q8_0 scale with code 1 decodes to that value."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    blocks = np.zeros((65536, 34), np.uint8)
    blocks[:, 0] = h & 0xFF
    blocks[:, 1] = h >> 8
    blocks[:, 2:] = 1
    got = gpu_dequant(blocks.reshape(-1), Q8).reshape(65536, 32)
    exp = h.view(np.float16).astype(np.float32)
    for j in (0, 31):
        assert_bits_equal_nan_aware(got[:, j], exp)


@pytest.mark.parametrize("t", [Q4, Q5, Q8])
def test_dequant_bit_exact(t, gold_dequant):
    blocks = fwgpu.synth_matrix(t, 64, 512, seed=40 + t, subnormal_every=3)
    assert_bits_equal_nan_aware(gpu_dequant(blocks, t), fw_cpu.dequant(blocks, t))
    if t in (Q5, Q8):
        fb = gold_dequant[f"blocks_{t}"]
        assert_bits_equal_nan_aware(gpu_dequant(fb, t), gold_dequant[f"getrow_{t}"])


@pytest.mark.parametrize("t", [Q4, Q5, Q8, F32])
def test_get_row_bit_exact(t):
    rows, cols = 37, 288
    if t == F32:
        w = fwgpu.randn(3, rows * cols)
        exp = w.reshape(rows, cols)[29]
        wb = w.view(np.uint8)
    else:
        wb = fwgpu.synth_matrix(t, rows, cols, seed=9)
        exp = fw_cpu.dequant(wb, t).reshape(rows, cols)[29]
    d, o = DB.from_array(wb), DB(cols * 4)
    ops.get_row(d, t, cols, 29, o)
    assert np.array_equal(bits(o.to_array(np.float32)), bits(exp))


def run_qmv(w, t, x, rows, x_offset=0):
    xb = np.zeros(x.size + x_offset, np.float32)
    xb[x_offset:] = x
    dw, dx, dy = DB.from_array(w), DB.from_array(xb), DB(rows * 4)

    class View:   # x at a byte offset inside its buffer (unaligned-x path)
        ptr = dx.ptr + 4 * x_offset
    ops.quant_matvec(dw, t, View if x_offset else dx, dy, x.size, rows)
    return dy.to_array(np.float32)


def check_close(y, ref, bound=None):
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= ATOL + RTOL * np.abs(ref)), f"max err {err.max()}"
    if bound is not None:
        assert np.all(err <= 2e-5 * bound + 1e-30), f"max err/bound {np.max(err / (bound + 1e-30))}"


def abs_bound(w, t, x, rows):
    W = fw_cpu.dequant(w, t).reshape(rows, -1) if t != F32 else w.view(np.float32).reshape(rows, -1)
    return np.abs(W).astype(np.float64) @ np.abs(x).astype(np.float64)


@pytest.mark.parametrize("case", gs.MATVEC_CASES, ids=lambda c: gs.matvec_key(*c))
def test_quant_matvec_vs_reference_fixtures(case, gold_matvec):
    t, rows, cols = case
    w, x = gs.matvec_weights(t, rows, cols), gs.matvec_x(t, rows, cols)
    y = run_qmv(w, t, x, rows)
    check_close(y, gold_matvec[gs.matvec_key(t, rows, cols)], abs_bound(w, t, x, rows))


@pytest.mark.parametrize("shape", [(4096, 4096), (14336, 4096), (4096, 14336)])
def test_quant_matvec_q4_0_microbench_shapes(shape):
    rows, cols = shape
    w = fwgpu.synth_matrix(Q4, rows, cols, seed=rows + cols)
    x = fwgpu.randn(cols, cols)
    fw_cpu.set_threads(16)
    rc, ref = fw_cpu.quant_matvec(w, Q4, x, rows)
    assert rc == 0
    check_close(run_qmv(w, Q4, x, rows), ref, abs_bound(w, Q4, x, rows))


@pytest.mark.parametrize("t", [Q4, Q5, Q8, F32])
@pytest.mark.parametrize("shape", [(1, 32), (7, 96), (13, 288), (5, 768), (66, 1024)])
def test_quant_matvec_ragged_shapes(t, shape):
    rows, cols = shape
    x = fwgpu.randn(5 + cols, cols)
    if t == F32:
        w = fwgpu.randn(6 + rows, rows * cols).view(np.uint8)
    else:
        w = fwgpu.synth_matrix(t, rows, cols, seed=rows * cols + t, subnormal_every=7)
    rc, ref = fw_cpu.quant_matvec(w if t != F32 else w.view(np.float32), t, x, rows)
    assert rc == 0
    b = abs_bound(w, t, x, rows)
    check_close(run_qmv(w, t, x, rows), ref, b)
    check_close(run_qmv(w, t, x, rows, x_offset=1), ref, b)       # x not 16-byte aligned


def test_quant_matvec_kat_64():                                    # test_runner.c:161-178
    blk = np.zeros(34, np.uint8)
    blk[1] = 0x3C
    blk[2:] = 2
    assert run_qmv(blk, Q8, np.ones(32, np.float32), 1)[0] == 64.0


def test_quant_matvec_q4_0_one_hot_and_linearity():
    rows, cols = 64, 4096
    w = fwgpu.synth_matrix(Q4, rows, cols, seed=77)
    W = fw_cpu.dequant(w, Q4).reshape(rows, cols)
    for j in (0, 33, 4095):
        e = np.zeros(cols, np.float32)
        e[j] = 1
        assert np.array_equal(bits(run_qmv(w, Q4, e, rows)), bits(W[:, j]))
    x = fwgpu.randn(8, cols)
    assert np.array_equal(bits(run_qmv(w, Q4, x * np.float32(2), rows)), bits(run_qmv(w, Q4, x, rows) * 2))


@pytest.mark.parametrize("n", gs.NORM_SIZES)
def test_rms_norm_bit_exact(n, gold_ops):
    x, w = gs.norm_inputs(n)
    dx, dw, do = DB.from_array(x), DB.from_array(w), DB(n * 4)
    ops.rms_norm(dx, dw, do, n, gs.NORM_EPS)
    assert np.array_equal(bits(do.to_array(np.float32)), bits(gold_ops[f"rmsnorm_{n}"]))
    ops.tensor_rms_norm(dx, dw, do, n, gs.NORM_EPS)
    assert np.array_equal(bits(do.to_array(np.float32)), bits(gold_ops[f"rmsnorm_{n}"]))


@pytest.mark.parametrize("case", gs.ROPE_CASES)
def test_rope_bit_exact(case, gold_ops):
    pos, nh, hd, nctx, base, neox = case
    cos = np.zeros(nctx * hd // 2, np.float32)
    sin = np.zeros_like(cos)
    fwgpu.host_lib().fwh_rope_tables(cos.ctypes.data_as(fwgpu.fp), sin.ctypes.data_as(fwgpu.fp), nctx, hd, base)
    qk = DB.from_array(gs.rope_input(nh, hd))
    ops.rope_apply(qk, pos, nh, hd, DB.from_array(cos), DB.from_array(sin), neox)
    assert np.array_equal(bits(qk.to_array(np.float32)), bits(gold_ops[f"rope_{pos}_{nh}_{hd}_{int(base)}_{neox}"]))


def ulps(a, b):
    a = bits(a).astype(np.int64)
    b = bits(b).astype(np.int64)
    a = np.where(a & 0x80000000, 0x80000000 - a, a)
    b = np.where(b & 0x80000000, 0x80000000 - b, b)
    return np.abs(a - b)


def test_silu_within_one_ulp(gold_ops):
    """expf is the only libm call: the GPU's is correctly rounded, glibc's is within 0.502 ulp."""
    x = gs.silu_input()
    dx, do = DB.from_array(x), DB(x.size * 4)
    ops.tensor_silu(dx, do, x.size)
    assert ulps(do.to_array(np.float32), gold_ops["silu"]).max() <= 1
    g, u = fwgpu.randn(1, 14336, 3.0), fwgpu.randn(2, 14336)
    dg, du, dh = DB.from_array(g), DB.from_array(u), DB(14336 * 4)
    ops.silu_mul(dg, du, dh, 14336)
    assert ulps(dh.to_array(np.float32), fw_cpu.silu(g) * u).max() <= 2


def test_tensor_add_and_matvec_f32():
    a, b = fwgpu.randn(1, 1000), fwgpu.randn(2, 1000)
    da, db, do = DB.from_array(a), DB.from_array(b), DB(4000)
    ops.tensor_add(da, db, do, 1000)
    assert np.array_equal(bits(do.to_array(np.float32)), bits(a + b))
    W = np.array([[1, 2, 3, 4, 5], [2, 0, 1, -1, 3], [-1, 1, -1, 1, 0]], np.float32)   # test_runner.c:250-265
    x = np.array([1, -2, 3, -4, 5], np.float32)
    dy = DB(12)
    ops.tensor_matvec_f32(DB.from_array(W), DB.from_array(x), dy, 3, 5)
    assert np.allclose(dy.to_array(np.float32), [15, 24, -10], atol=1e-4)


def test_argmax_reference_cases(gold_ops):
    got = []
    for c in gs.argmax_cases():
        dx, do = DB.from_array(c), DB(4)
        ops.argmax(dx, c.size, do)
        got.append(int(do.to_array(np.uint32)[0]))
    assert got == gold_ops["argmax"].tolist()
    for n in (1, 255, 256, 257, 2048 * 256 + 3):   # one block ... many blocks
        x = fwgpu.randn(n, n)
        x[n // 3] = 50.0
        x[n - 1] = 50.0
        dx, do = DB.from_array(x), DB(4)
        ops.argmax(dx, n, do)
        assert int(do.to_array(np.uint32)[0]) == fw_cpu.argmax(x)


@pytest.mark.parametrize("cfg", [(6, 6, 48, 0), (6, 6, 48, 143), (8, 2, 32, 30), (32, 8, 128, 767),
                                 (64, 8, 128, 382), (16, 8, 64, 1000), (32, 8, 128, 5000),
                                 # head_dim 80/96/256 and groups 3/6/7/12 (phi-2, phi-3, gemma, qwen2 shapes)
                                 (32, 32, 80, 300), (32, 32, 96, 200), (8, 1, 256, 150), (16, 16, 256, 90),
                                 (14, 2, 64, 400), (12, 2, 128, 77), (28, 4, 128, 257), (12, 4, 96, 33),
                                 (24, 2, 80, 64)],
                         ids=lambda c: "h{}_kv{}_hd{}_pos{}".format(*c))
def test_attention_vs_oracle(cfg):
    n_head, n_kv, hd, pos = cfg
    n_ctx = pos + 3
    rng = np.random.default_rng(pos + hd)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    k = rng.standard_normal(n_ctx * n_kv * hd).astype(np.float32)
    v = rng.standard_normal(n_ctx * n_kv * hd).astype(np.float32)
    out = DB(n_head * hd * 4)
    ops.attention(DB.from_array(q), DB.from_array(k), DB.from_array(v), out, n_head, n_kv, hd, n_ctx, pos)
    ref = fw_cpu.attention_core(q, k, v, n_head, n_kv, hd, pos)
    check_close(out.to_array(np.float32), ref)
    assert np.max(np.abs(out.to_array(np.float32) - ref)) < 1e-5
