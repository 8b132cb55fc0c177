"""Architecture variants of the RMSNorm / gated-FFN block on the GPU, each held
to the oracle (whose forward for each is pinned bit-exactly to the reference by
a golden model fixture) on every decode path: the persistent step kernel, the
per-phase kernels and the batched prefill.

qwen2: llama's block plus F32 biases on the q, k and v projections
(attention.c:114-126 via linear.c:214-221), added before RoPE, and the RoPE
base the config loader raises to 1e6 (model_config.c:161-168).

gemma: the gated FFN with the tanh GELU (ffn.c:33-42, model_config.c:170-176),
embedding rows times sqrt(n_embd) (transformer.c:179-182) and, with no
output.weight in the file, the lm-head read from token_embd
(transformer.c:309-316).  The erf GELU (ffn.c:27-31) is run through the same
kernels by selecting it in the config.

phi2: LayerNorm with biases (norm.c:18-40), parallel residual
(transformer.c:232-252), plain FFN with the tanh GELU (ffn.c:108-171), NEOX
RoPE (rope.c:44-51) and the output-projection bias (attention.c:106-107), on
the explicit per-phase step (the persistent kernel serves the RMSNorm / gated /
sequential / pairwise-RoPE block only) and in the batched prefill.  Config overrides on the same file run the
remaining combinations: sequential LayerNorm, RMSNorm, pairwise RoPE, and the
plain FFN's relu / silu / erf-GELU activations.

Bar: logits and the residual stream within max-abs 2e-3 / rel 1e-3,
identical greedy tokens."""
import os

import numpy as np
import pytest

import fw_cpu
import fwgpu
import golden_specs as gs
from conftest import gold_model

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-3, 1e-3
Q4, Q8 = fwgpu.GGML_Q4_0, fwgpu.GGML_Q8_0


def close(got, exp, what):
    err = np.abs(got.astype(np.float64) - exp.astype(np.float64))
    bad = ~(err <= ATOL + RTOL * np.abs(exp))                  # NaN counts as out of tolerance
    assert not bad.any(), f"{what}: {bad.sum()} elements out of tolerance, max err {err.max():.3g}"
    return float(err.max())


class env:
    def __init__(self, **kw):
        self.kw = kw

    def __enter__(self):
        for k, v in self.kw.items():
            os.environ[k] = v

    def __exit__(self, *a):
        for k in self.kw:
            del os.environ[k]


def qwen2_q4(seed=21):
    # head_dim 64, GQA group 4, Q4_0 layers (the persistent kernel's shape class)
    return fwgpu.spec(512, 1536, 2, 8, 2, 2048, 96, 10000.0, linear_type=Q4, seed=seed, arch="qwen2")


@pytest.mark.parametrize("persistent", [True, False], ids=["persistent", "per_phase"])
def test_qwen2_decode_matches_oracle(persistent):
    fw_cpu.set_threads(8)
    with env(**({} if persistent else {"FORWORD_GPU_MEGAKERNEL": "0"})):
        with fwgpu.HostModel(synth=qwen2_q4()) as host, fwgpu.GpuModel(host) as gm, \
                fw_cpu.OracleModel(host) as om:
            assert host.cfg.use_qkv_bias == 1 and host.cfg.rope_freq_base == 1e6
            assert gm.persistent == persistent
            toks = np.random.default_rng(4).integers(3, host.cfg.n_vocab, 10)
            for pos, t in enumerate(toks):
                lg, ref = gm.forward(int(t), pos), om.forward(int(t), pos)
                close(lg, ref, f"logits at position {pos}")
                assert fw_cpu.argmax(lg) == fw_cpu.argmax(ref)
                if pos in (0, 9):
                    close(gm.layer_trace().reshape(-1), om.trace().reshape(-1), f"residual stream at {pos}")
            k, v = gm.kv_read(host.cfg.n_layer - 1, 0, len(toks))
            kr, vr = om.kv(host.cfg.n_layer - 1, 0)
            close(k[0], kr, "post-RoPE K row (bias before RoPE)")
            close(v[0], vr, "V row (bias)")


def test_qwen2_fixture_per_phase_matches_reference():
    """The reference-generated qwen2 fixture on the per-phase kernels (the
    model-level tests run it on the persistent kernel): logits at the recorded
    forwards and the greedy continuation."""
    prompt = gs.prompt("qwen2")
    gold = gold_model("qwen2")
    m = gs.MODELS["qwen2"]
    with env(FORWORD_GPU_MEGAKERNEL="0"):
        with fwgpu.HostModel(synth=m["spec"](), max_ctx=m["max_ctx"]) as host, fwgpu.GpuModel(host) as gm:
            assert not gm.persistent
            toks = gold["tokens"]
            for f in range(gs.n_forwards("qwen2")):
                lg = gm.forward(int(toks[f]), f)
                assert fw_cpu.argmax(lg) == int(gold["stats"][f, 0]), f"greedy choice differs at forward {f}"
                if f in gs.logit_steps("qwen2"):
                    close(lg, gold[f"logits_{f}"], f"logits at forward {f}")
            got = gm.generate_greedy(prompt, m["n_gen"])
    assert np.array_equal(got, gold["tokens"][len(prompt):])


def test_qwen2_prefill_matches_oracle():
    """Batched prefill adds the bias in its RoPE/append kernel: last-token
    logits and every KV row against the oracle's token-by-token prefill."""
    fw_cpu.set_threads(8)
    with fwgpu.HostModel(synth=qwen2_q4(seed=22)) as host, fwgpu.GpuModel(host) as gm, \
            fw_cpu.OracleModel(host) as om:
        prompt = np.random.default_rng(6).integers(3, host.cfg.n_vocab, 40).astype(np.uint32)
        lg = gm.prefill(prompt)
        for pos, t in enumerate(prompt):
            ref = om.forward(int(t), pos)
        close(lg, ref, "prefill logits")
        assert fw_cpu.argmax(lg) == fw_cpu.argmax(ref)
        for layer in range(host.cfg.n_layer):
            k, v = gm.kv_read(layer, 0, len(prompt))
            for pos in (0, 17, len(prompt) - 1):
                kr, vr = om.kv(layer, pos)
                close(k[pos], kr, f"K row layer {layer} pos {pos}")
                close(v[pos], vr, f"V row layer {layer} pos {pos}")


def gemma_q4(seed=31):
    return fwgpu.spec(512, 1536, 2, 8, 2, 2048, 96, 10000.0, linear_type=Q4, seed=seed, arch="gemma")


@pytest.mark.parametrize("act", ["gelu_tanh", "gelu_erf"])
@pytest.mark.parametrize("persistent", [True, False], ids=["persistent", "per_phase"])
def test_gemma_decode_matches_oracle(persistent, act):
    fw_cpu.set_threads(8)
    with env(**({} if persistent else {"FORWORD_GPU_MEGAKERNEL": "0"})):
        with fwgpu.HostModel(synth=gemma_q4()) as host:
            assert host.cfg.act_type == 2 and host.cfg.embd_scale == np.float32(np.sqrt(512))
            if act == "gelu_erf":
                host.cfg.act_type = 1
            with fwgpu.GpuModel(host) as gm, fw_cpu.OracleModel(host) as om:
                assert gm.persistent == persistent
                toks = np.random.default_rng(8).integers(3, host.cfg.n_vocab, 10)
                for pos, t in enumerate(toks):
                    lg, ref = gm.forward(int(t), pos), om.forward(int(t), pos)
                    close(lg, ref, f"{act} logits at position {pos}")
                    assert fw_cpu.argmax(lg) == fw_cpu.argmax(ref)
                    if pos in (0, 9):
                        close(gm.layer_trace().reshape(-1), om.trace().reshape(-1), f"residual stream at {pos}")
                got = gm.generate_greedy(toks[:4].astype(np.uint32), 12)
                om_toks = om.generate_greedy(toks[:4].astype(np.uint32), 12)
                assert np.array_equal(got, om_toks)


def test_gemma_fixture_per_phase_matches_reference():
    prompt = gs.prompt("gemma")
    gold = gold_model("gemma")
    m = gs.MODELS["gemma"]
    with env(FORWORD_GPU_MEGAKERNEL="0"):
        with fwgpu.HostModel(synth=m["spec"](), max_ctx=m["max_ctx"]) as host, fwgpu.GpuModel(host) as gm:
            toks = gold["tokens"]
            for f in range(gs.n_forwards("gemma")):
                lg = gm.forward(int(toks[f]), f)
                assert fw_cpu.argmax(lg) == int(gold["stats"][f, 0]), f"greedy choice differs at forward {f}"
                if f in gs.logit_steps("gemma"):
                    close(lg, gold[f"logits_{f}"], f"logits at forward {f}")
            got = gm.generate_greedy(prompt, m["n_gen"])
    assert np.array_equal(got, gold["tokens"][len(prompt):])


def test_gemma_prefill_matches_oracle():
    fw_cpu.set_threads(8)
    with fwgpu.HostModel(synth=gemma_q4(seed=32)) as host, fwgpu.GpuModel(host) as gm, \
            fw_cpu.OracleModel(host) as om:
        prompt = np.random.default_rng(9).integers(3, host.cfg.n_vocab, 40).astype(np.uint32)
        lg = gm.prefill(prompt)
        for pos, t in enumerate(prompt):
            ref = om.forward(int(t), pos)
        close(lg, ref, "prefill logits")
        assert fw_cpu.argmax(lg) == fw_cpu.argmax(ref)


PHI2_OVERRIDES = {
    "phi2": {},
    "sequential_layernorm": {"parallel_res": 0},
    "rmsnorm": {"norm_type": 0},
    "pairwise_rope": {"rope_type": 0},
    "plain_relu": {"act_type": 3},
    "plain_silu": {"act_type": 0},
    "plain_gelu_erf": {"act_type": 1},
}


@pytest.mark.parametrize("variant", list(PHI2_OVERRIDES))
def test_phi2_family_matches_oracle(variant):
    fw_cpu.set_threads(8)
    sp = fwgpu.spec(512, 1536, 2, 8, 8, 2048, 96, 10000.0, linear_type=Q4, seed=41, arch="phi2")
    with fwgpu.HostModel(synth=sp) as host:
        c = host.cfg
        assert (c.norm_type, c.parallel_res, c.use_ffn_gate, c.rope_type, c.act_type) == (1, 1, 0, 1, 2)
        for k, v in PHI2_OVERRIDES[variant].items():
            setattr(host.cfg, k, v)
        with fwgpu.GpuModel(host) as gm, fw_cpu.OracleModel(host) as om:
            assert not gm.persistent
            toks = np.random.default_rng(12).integers(3, host.cfg.n_vocab, 10)
            for pos, t in enumerate(toks):
                lg, ref = gm.forward(int(t), pos), om.forward(int(t), pos)
                close(lg, ref, f"{variant} logits at position {pos}")
                assert fw_cpu.argmax(lg) == fw_cpu.argmax(ref)
                if pos in (0, 9):
                    close(gm.layer_trace().reshape(-1), om.trace().reshape(-1), f"residual stream at {pos}")
            k, v = gm.kv_read(host.cfg.n_layer - 1, 0, len(toks))
            for pos in (0, 9):
                kr, vr = om.kv(host.cfg.n_layer - 1, pos)
                close(k[pos], kr, f"K row at {pos}")
                close(v[pos], vr, f"V row at {pos}")
            got = gm.generate_greedy(toks[:4].astype(np.uint32), 12)
            assert np.array_equal(got, om.generate_greedy(toks[:4].astype(np.uint32), 12))
            # batched prefill of the same block: last logits and KV rows
            prompt = np.random.default_rng(15).integers(3, host.cfg.n_vocab, 33).astype(np.uint32)
            lg = gm.prefill(prompt)
            for pos, t in enumerate(prompt):
                ref = om.forward(int(t), pos)
            close(lg, ref, f"{variant} prefill logits")
            k, v = gm.kv_read(0, 0, len(prompt))
            for pos in (0, 32):
                kr, vr = om.kv(0, pos)
                close(k[pos], kr, f"prefill K row at {pos}")
                close(v[pos], vr, f"prefill V row at {pos}")


def test_neox_rope_on_gated_block_matches_oracle():
    """NEOX pairs on the llama block (config override): the per-phase step
    rotates after the QKV projection; the persistent kernel steps aside."""
    fw_cpu.set_threads(8)
    with fwgpu.HostModel(synth=qwen2_q4(seed=23)) as host:
        host.cfg.rope_type = 1
        with fwgpu.GpuModel(host) as gm, fw_cpu.OracleModel(host) as om:
            assert not gm.persistent
            toks = np.random.default_rng(13).integers(3, host.cfg.n_vocab, 8)
            for pos, t in enumerate(toks):
                close(gm.forward(int(t), pos), om.forward(int(t), pos), f"logits at position {pos}")


def test_phi2_fixture_prefill_and_greedy_match_reference():
    """The phi2 batched prefill and the greedy loop after it against the
    reference-generated fixture."""
    name = "phi2"
    gold = gold_model(name)
    m = gs.MODELS[name]
    prompt = gs.prompt(name)
    f = len(prompt) - 1
    with fwgpu.HostModel(synth=m["spec"](), max_ctx=m["max_ctx"]) as host, fwgpu.GpuModel(host) as gm:
        lg = gm.prefill(prompt)
        close(lg, gold[f"logits_{f}"], "prefill logits")
        got = gm.generate_greedy_batched(prompt, m["n_gen"])
    assert np.array_equal(got, gold["tokens"][len(prompt):])


# Head dims and GQA groups of real checkpoints the persistent kernel does not
# take (the per-phase step and the batched prefill run them): phi-2 hd 80,
# phi-3 hd 96, gemma hd 256 (group 8), qwen2 groups 6 and 7.
SHAPES_HD_GROUP = {
    "llama_hd80_g1": (640, 1024, 2, 8, 8, 1000, "llama"),
    "llama_hd96_g3": (1152, 1536, 2, 12, 4, 1000, "llama"),
    "gemma_hd256_g8": (2048, 2048, 1, 8, 1, 1000, "gemma"),
    "qwen2_hd64_g7": (896, 1536, 2, 14, 2, 1000, "qwen2"),
    "qwen2_hd128_g6": (1536, 2048, 1, 12, 2, 1000, "qwen2"),
    "phi2_hd80_g1": (640, 1024, 2, 8, 8, 1000, "phi2"),
}


@pytest.mark.parametrize("name", list(SHAPES_HD_GROUP))
def test_head_dims_and_groups_match_oracle(name):
    e, f, L, h, kv, v, arch = SHAPES_HD_GROUP[name]
    fw_cpu.set_threads(8)
    sp = fwgpu.spec(e, f, L, h, kv, v, 64, 10000.0, seed=51, arch=arch)
    with fwgpu.HostModel(synth=sp) as host, fwgpu.GpuModel(host) as gm, fw_cpu.OracleModel(host) as om:
        assert host.cfg.head_dim == e // h
        toks = np.random.default_rng(14).integers(3, v, 20).astype(np.uint32)
        for pos, t in enumerate(toks[:6]):
            lg, ref = gm.forward(int(t), pos), om.forward(int(t), pos)
            close(lg, ref, f"{name} logits at position {pos}")
        lg = gm.prefill(toks)                       # batched where the block allows it
        for pos, t in enumerate(toks):
            ref = om.forward(int(t), pos)
        close(lg, ref, f"{name} prefill logits")
        assert fw_cpu.argmax(lg) == fw_cpu.argmax(ref)


def test_gpt2_matches_oracle():
    """GPT-2 block (model_config.c:197-207): learned position rows added to the
    embedding (transformer.c:188-205), one [q | k | v] projection with its bias
    (attention.c:68-96), no RoPE, LayerNorm, plain erf-GELU FFN with up/down
    biases (ffn.c:127-168), head tied to token_embd: decode, prefill, greedy."""
    fw_cpu.set_threads(8)
    sp = fwgpu.spec(512, 2048, 2, 8, 8, 2048, 96, 10000.0, linear_type=Q4, seed=61, arch="gpt2")
    with fwgpu.HostModel(synth=sp) as host, fwgpu.GpuModel(host) as gm, fw_cpu.OracleModel(host) as om:
        c = host.cfg
        assert (c.arch, c.rope_type, c.norm_type, c.use_ffn_gate, c.act_type) == (1, 2, 1, 0, 1)
        assert not gm.persistent
        toks = np.random.default_rng(16).integers(3, c.n_vocab, 10)
        for pos, t in enumerate(toks):
            lg, ref = gm.forward(int(t), pos), om.forward(int(t), pos)
            close(lg, ref, f"logits at position {pos}")
            assert fw_cpu.argmax(lg) == fw_cpu.argmax(ref)
            if pos in (0, 9):
                close(gm.layer_trace().reshape(-1), om.trace().reshape(-1), f"residual stream at {pos}")
        got = gm.generate_greedy(toks[:4].astype(np.uint32), 12)
        assert np.array_equal(got, om.generate_greedy(toks[:4].astype(np.uint32), 12))
        prompt = np.random.default_rng(17).integers(3, c.n_vocab, 40).astype(np.uint32)
        lg = gm.prefill(prompt)
        for pos, t in enumerate(prompt):
            ref = om.forward(int(t), pos)
        close(lg, ref, "prefill logits")
        k, v = gm.kv_read(1, 0, len(prompt))
        kr, vr = om.kv(1, 39)
        close(k[39], kr, "prefill K row (no RoPE)")
        close(v[39], vr, "prefill V row")
