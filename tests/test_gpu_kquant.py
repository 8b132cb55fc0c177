"""Q4_K and Q6_K (256-value super-blocks, quant.c:63-189) on the GPU: dequant
bit-exact to the reference's decoders (golden fixtures written by the compiled
reference), quant_matvec within tolerance of the reference's outputs
(quant_matvec.c:231-261), and a Q4_K/Q6_K model equal to the oracle: logits
within max-abs 2e-3 / rel 1e-3, identical greedy tokens, and the batched
prefill on the same model, on the persistent step kernel (Q4_K linears in
place, a Q6_K lm-head from its re-laid-out copy) and on the per-phase kernels."""
import numpy as np
import pytest

import fw_cpu
import fwgpu
import golden_specs as gs
from conftest import kernel_choice
from fwgpu import DeviceBuffer as DB, ops

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-3, 1e-3


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def gpu_dequant(blocks, t):
    n = blocks.size // fwgpu.BLOCK_BYTES[t] * fwgpu.BLOCK_VALUES[t]
    d, o = DB.from_array(blocks), DB(n * 4)
    ops.dequant(d, t, o, n)
    return o.to_array(np.float32)


def check_close(y, ref, what):
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    bad = ~(err <= ATOL + RTOL * np.abs(ref))                  # NaN counts as out of tolerance
    assert not bad.any(), f"{what}: {bad.sum()} out of tolerance, max err {err.max():.3g}"


@pytest.mark.parametrize("t", gs.KQ_TYPES)
def test_dequant_bit_exact_vs_reference(t, gold_kquant):
    blocks = gold_kquant[f"blocks_{t}"]
    got, exp = gpu_dequant(blocks, t), gold_kquant[f"getrow_{t}"]
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got)[~nan], bits(exp)[~nan])
    w = fwgpu.synth_matrix(t, 16, 1024, seed=60 + t)
    assert np.array_equal(bits(gpu_dequant(w, t)), bits(fw_cpu.dequant(w, t)))


@pytest.mark.parametrize("t", gs.KQ_TYPES)
def test_get_row_bit_exact(t):
    rows, cols = 9, 512
    w = fwgpu.synth_matrix(t, rows, cols, seed=70 + t)
    d, o = DB.from_array(w), DB(cols * 4)
    ops.get_row(d, t, cols, 5, o)
    assert np.array_equal(bits(o.to_array(np.float32)), bits(fw_cpu.dequant(w, t).reshape(rows, cols)[5]))


@pytest.mark.parametrize("case", gs.KQ_MATVEC_CASES, ids=lambda c: gs.matvec_key(*c))
def test_quant_matvec_vs_reference(case, gold_kquant):
    t, rows, cols = case
    w, x = gs.matvec_weights(t, rows, cols), gs.matvec_x(t, rows, cols)
    dw, dx, dy = DB.from_array(w), DB.from_array(x), DB(rows * 4)
    ops.quant_matvec(dw, t, dx, dy, cols, rows)
    ref = gold_kquant[gs.matvec_key(t, rows, cols)]
    y = dy.to_array(np.float32)
    W = fw_cpu.dequant(w, t).reshape(rows, cols).astype(np.float64)
    bound = np.abs(W) @ np.abs(x.astype(np.float64))
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= 2e-5 * bound + 1e-30), f"max err/bound {np.max(err / (bound + 1e-30))}"


def kq_spec(name="q4k"):
    """Q4_K linears and embedding with a Q6_K output (the Q4_K_M layout's two
    types); the same layers with a Q8_0 output; Q4_0 layers with a Q6_K output
    (llama.cpp's Q4_0 files keep the output Q6_K).  "q4k_odd": column slices
    padded to whole super-blocks (768 = 3 x 256 columns, n_ff 1280 = 5 x 256)."""
    if name == "q4k":
        return fwgpu.spec(512, 1024, 2, 8, 2, 2000, 96, 10000.0, linear_type=gs.Q4K, embd_type=gs.Q4K,
                          output_type=gs.Q6K, seed=1212)
    if name == "q4k_q8":
        return fwgpu.spec(512, 1024, 2, 8, 2, 2000, 96, 10000.0, linear_type=gs.Q4K, embd_type=gs.Q4K,
                          output_type=fwgpu.GGML_Q8_0, seed=1214)
    if name == "q4_0_q6k":
        return fwgpu.spec(512, 1024, 2, 8, 2, 2000, 96, 10000.0, linear_type=fwgpu.GGML_Q4_0,
                          embd_type=fwgpu.GGML_Q4_0, output_type=gs.Q6K, seed=1215)
    assert name == "q4k_odd"
    return fwgpu.spec(768, 1280, 2, 12, 4, 1500, 96, 10000.0, linear_type=gs.Q4K, embd_type=gs.Q6K,
                      output_type=gs.Q6K, seed=1216)


@pytest.mark.parametrize("persistent", [True, False], ids=["persistent", "per_phase"])
@pytest.mark.parametrize("name", ["q4k", "q4k_q8", "q4_0_q6k", "q4k_odd"])
def test_kquant_model_matches_oracle(name, persistent):
    """Per-token decode, the device-resident greedy loop and the batched prefill
    against the oracle, on the persistent step kernel and on the per-phase kernels."""
    prompt = np.random.default_rng(12).integers(3, 1500, 10).astype(np.uint32)
    with fwgpu.HostModel(synth=kq_spec(name)) as host, fw_cpu.OracleModel(host) as om:
        with kernel_choice(persistent), fwgpu.GpuModel(host) as gm:
            assert gm.persistent == persistent
            toks = list(prompt)
            for f in range(len(prompt) + 5):
                exp = om.forward(int(toks[f]), f)
                got = gm.forward(int(toks[f]), f)
                check_close(got, exp, f"logits at forward {f}")
                assert fw_cpu.argmax(got) == fw_cpu.argmax(exp)
                if f + 1 >= len(toks):
                    toks.append(fw_cpu.argmax(exp))
            check_close(gm.layer_trace().reshape(-1), om.trace().reshape(-1), "residual stream")
            ref_gen = np.array(toks[len(prompt):len(prompt) + 6], np.uint32)
        with kernel_choice(persistent), fwgpu.GpuModel(host) as gm:
            assert np.array_equal(gm.generate_greedy(prompt, 6), ref_gen)
        with kernel_choice(persistent), fwgpu.GpuModel(host) as gm:
            lg = gm.prefill(prompt)
            assert fw_cpu.argmax(lg) == int(ref_gen[0])
            assert np.array_equal(gm.generate_greedy_batched(prompt, 6), ref_gen)


def mixed_spec():
    """The reference's own model layout (tensors.txt, a Q4_K_M file): Q4_K linears with
    attn_v and ffn_down Q6_K on every other layer, n_ff an odd number of super-blocks
    (1280 = 5 x 256), Q6_K output."""
    return fwgpu.spec(512, 1280, 4, 8, 2, 2000, 96, 10000.0, linear_type=gs.Q4K, embd_type=gs.Q4K,
                      output_type=gs.Q6K, seed=1313, mix_type=gs.Q6K)


@pytest.mark.parametrize("persistent", [True, False], ids=["persistent", "per_phase"])
def test_mixed_type_layers_match_oracle(persistent):
    """Per-tensor types that change inside a layer and from layer to layer:
    per-token decode, the device-resident greedy loop and the batched prefill.
    On the persistent kernel the Q6_K attn_v rows run as a second GEMV of the
    QKV phase and the Q6_K ffn_down layers with their own type."""
    prompt = np.random.default_rng(13).integers(3, 2000, 10).astype(np.uint32)
    with fwgpu.HostModel(synth=mixed_spec()) as host, fw_cpu.OracleModel(host) as om:
        assert host.tensor("blk.0.attn_v.weight").ggml_type == gs.Q6K
        assert host.tensor("blk.1.attn_v.weight").ggml_type == gs.Q4K
        assert host.tensor("blk.2.ffn_down.weight").ggml_type == gs.Q6K
        assert host.tensor("blk.3.ffn_down.weight").ggml_type == gs.Q4K
        with kernel_choice(persistent), fwgpu.GpuModel(host) as gm:
            assert gm.persistent == persistent
            toks = list(prompt)
            for f in range(len(prompt) + 5):
                exp = om.forward(int(toks[f]), f)
                got = gm.forward(int(toks[f]), f)
                check_close(got, exp, f"logits at forward {f}")
                assert fw_cpu.argmax(got) == fw_cpu.argmax(exp)
                if f + 1 >= len(toks):
                    toks.append(fw_cpu.argmax(exp))
            check_close(gm.layer_trace().reshape(-1), om.trace().reshape(-1), "residual stream")
            ref_gen = np.array(toks[len(prompt):len(prompt) + 6], np.uint32)
        with kernel_choice(persistent), fwgpu.GpuModel(host) as gm:
            assert np.array_equal(gm.generate_greedy(prompt, 6), ref_gen)
        with kernel_choice(persistent), fwgpu.GpuModel(host) as gm:
            lg = gm.prefill(prompt)
            assert fw_cpu.argmax(lg) == int(ref_gen[0])
            assert np.array_equal(gm.generate_greedy_batched(prompt, 6), ref_gen)


@pytest.mark.slow
@pytest.mark.parametrize("mix", [False, True], ids=["q4_k", "q4_k_m"])
def test_8b_shape_kquant_persistent_vs_oracle(mix):
    """Llama-3-8B shape with Q4_K linears and embedding and a Q6_K lm-head (and the
    Q4_K_M layout: attn_v / ffn_down Q6_K in the even layers), on the persistent step
    kernel: 8 prompt tokens and 8 greedy tokens identical to the oracle run
    row-parallel on the host, and the last forward's logits within tolerance."""
    sp = fwgpu.spec_8b(n_ctx=64, linear_type=gs.Q4K, embd_type=gs.Q4K, output_type=gs.Q6K,
                       mix_type=gs.Q6K if mix else 0)
    prompt = np.random.default_rng(9).integers(3, 128256, 8).astype(np.uint32)
    fw_cpu.set_threads(16)
    with fwgpu.HostModel(synth=sp) as host:
        with kernel_choice(True), fwgpu.GpuModel(host) as gm:
            assert gm.persistent
            got = gm.generate_greedy(prompt, 8)
            lg = gm.forward(int(got[-1]), len(prompt) + 7)
        with fw_cpu.OracleModel(host) as om:
            exp = om.generate_greedy(prompt, 8)
            ref = om.forward(int(exp[-1]), len(prompt) + 7)
    assert np.array_equal(got, exp), (got, exp)
    check_close(lg, ref, "8B K-quant logits")
