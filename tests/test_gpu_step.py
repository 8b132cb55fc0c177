"""The persistent token-step kernel (one cooperative launch runs whole
transformer_forward steps, transformer.c:149-326, plus the greedy pick,
sampler.c:28-32) against the oracle and against the per-phase kernels.

Shapes cover every attention variant the kernel instantiates (head_dim 32 /
64 / 128, GQA group 1 / 2 / 4 / 8, and groups 3 / 6 / 7 walked in sub-groups), every weight type for the layer linears
and the lm-head, column slices of 1..64 block pairs, and workgroups that own
no rows.  Bar: logits and the residual stream within max-abs 2e-3 / rel 1e-3,
identical greedy tokens."""
import os

import numpy as np
import pytest

import fw_cpu
import fwgpu
import golden_specs as gs

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-3, 1e-3
Q4, Q5, Q8 = fwgpu.GGML_Q4_0, fwgpu.GGML_Q5_0, fwgpu.GGML_Q8_0

# name: (n_embd, n_ff, n_layer, n_head, n_head_kv, n_vocab, n_ctx, linear, embd, output)
SHAPES = {
    "hd64_g4_q4": (512, 1536, 2, 8, 2, 2048, 96, Q4, Q8, Q8),
    "hd128_g1_q5": (1024, 2816, 2, 8, 8, 3000, 64, Q5, Q5, Q5),
    "hd64_g8_q8": (1024, 2048, 2, 16, 2, 1536, 80, Q8, Q8, Q4),
    "hd32_g2_q4": (256, 768, 3, 8, 4, 1000, 160, Q4, Q4, Q5),
    "hd64_g1_wide": (256, 16448, 1, 4, 4, 512, 32, Q4, Q8, Q8),     # 257 pairs per down row: 64-pair slices
    # groups that are not powers of two (qwen2 7B: 7, 1.5B: 6) split into sub-group units
    "hd128_g7_q4": (1792, 2048, 2, 14, 2, 1000, 64, Q4, Q8, Q8),
    "hd64_g6_q8": (768, 1536, 2, 12, 2, 1000, 64, Q8, Q8, Q8),
    "hd64_g3_q5": (768, 1536, 2, 12, 4, 1000, 64, Q5, Q8, Q4),
}


def spec_of(name, seed=11):
    e, f, L, h, kv, v, ctx, lt, et, ot = SHAPES[name]
    return fwgpu.spec(e, f, L, h, kv, v, ctx, 10000.0, linear_type=lt, embd_type=et, output_type=ot, seed=seed)


def close(got, exp, what):
    err = np.abs(got.astype(np.float64) - exp.astype(np.float64))
    bad = ~(err <= ATOL + RTOL * np.abs(exp))                  # NaN counts as out of tolerance
    assert not bad.any(), f"{what}: {bad.sum()} elements out of tolerance, max err {err.max():.3g}"
    return float(err.max())


class per_phase_kernels:
    """Within the block, new GpuModel handles use one kernel per phase."""

    def __enter__(self):
        os.environ["FORWORD_GPU_MEGAKERNEL"] = "0"

    def __exit__(self, *a):
        del os.environ["FORWORD_GPU_MEGAKERNEL"]


@pytest.mark.parametrize("name", list(SHAPES))
def test_persistent_step_matches_oracle(name):
    fw_cpu.set_threads(8)
    with fwgpu.HostModel(synth=spec_of(name)) as host, fwgpu.GpuModel(host) as gm, \
            fw_cpu.OracleModel(host) as om:
        assert gm.persistent, "the persistent step kernel should run for this shape"
        toks = np.random.default_rng(3).integers(3, host.cfg.n_vocab, 12)
        for pos, t in enumerate(toks):
            lg, ref = gm.forward(int(t), pos), om.forward(int(t), pos)
            close(lg, ref, f"{name} logits at position {pos}")
            assert fw_cpu.argmax(lg) == fw_cpu.argmax(ref)
            if pos in (0, 11):
                close(gm.layer_trace().reshape(-1), om.trace().reshape(-1), f"{name} residual stream at {pos}")
        k, v = gm.kv_read(host.cfg.n_layer - 1, 0, len(toks))
        kr, vr = om.kv(host.cfg.n_layer - 1, 0)
        close(k[0], kr, f"{name} post-RoPE K row")
        close(v[0], vr, f"{name} V row")


@pytest.mark.parametrize("name,n_gen", [("hd64_g4_q4", 60), ("hd32_g2_q4", 140)])
def test_persistent_greedy_matches_oracle(name, n_gen):
    """Prompt + greedy tokens (148 forwards: three launches of up to 64 steps)
    and a decode() continuation, against the oracle's greedy loop."""
    fw_cpu.set_threads(8)
    n_prompt = 9
    with fwgpu.HostModel(synth=spec_of(name, seed=5)) as host:
        prompt = np.random.default_rng(9).integers(3, host.cfg.n_vocab, n_prompt).astype(np.uint32)
        with fw_cpu.OracleModel(host) as om:
            exp = om.generate_greedy(prompt, n_gen)
        with fwgpu.GpuModel(host) as gm:
            assert gm.persistent
            got = gm.generate_greedy(prompt, n_gen - 20)
            more = gm.decode(20)
    assert np.array_equal(np.concatenate([got, more]), exp), (got, more, exp)


def test_persistent_equals_per_phase_kernels():
    """Same model through both step implementations: close logits and residual
    streams, identical greedy tokens."""
    m = gs.MODELS["gqa"]
    toks = [3, 99, 512, 7, 7, 800, 1, 42]
    with fwgpu.HostModel(synth=m["spec"]()) as host:
        with fwgpu.GpuModel(host) as gm:
            assert gm.persistent
            a_logits = [gm.forward(t, i) for i, t in enumerate(toks)]
            a_trace = gm.layer_trace()
            a_tokens = gm.generate_greedy(toks[:3], 61)
        with per_phase_kernels(), fwgpu.GpuModel(host) as em:
            assert not em.persistent
            b_logits = [em.forward(t, i) for i, t in enumerate(toks)]
            b_trace = em.layer_trace()
            b_tokens = em.generate_greedy(toks[:3], 61)
    for i, (a, b) in enumerate(zip(a_logits, b_logits)):
        close(a, b, f"logits at position {i}")
    close(a_trace.reshape(-1), b_trace.reshape(-1), "residual stream")
    assert np.array_equal(a_tokens, b_tokens)


def test_persistent_forward_after_greedy_and_errors():
    """Host-driven forwards after a device-resident loop, argument errors
    leave the handle usable, prefill positions skip the lm-head."""
    with fwgpu.HostModel(synth=spec_of("hd64_g4_q4")) as host, fwgpu.GpuModel(host) as gm, \
            fw_cpu.OracleModel(host) as om:
        assert gm.persistent
        prompt = np.array([5, 6, 7, 8], np.uint32)
        first = gm.generate_greedy(prompt, 1)
        for p, t in enumerate(prompt):
            ref = om.forward(int(t), p)
        assert first[0] == fw_cpu.argmax(ref)
        assert not gm.forward_raw(0, host.n_ctx)
        assert "exceeds" in fwgpu.last_error()
        assert not gm.forward_raw(host.cfg.n_vocab, 0)
        nxt = gm.forward_argmax(int(first[0]), len(prompt))
        assert nxt == fw_cpu.argmax(om.forward(int(first[0]), len(prompt)))


@pytest.mark.parametrize("persistent", [True, False], ids=["persistent", "per_phase"])
def test_decode_from_after_kv_write_matches_oracle(persistent):
    """decode_from right after kv_write has filled the whole cache and a forward:
    the steps it queues start at the token and position the call names, also
    when it only queues them and decode continues the loop."""
    fw_cpu.set_threads(8)
    with fwgpu.HostModel(synth=spec_of("hd64_g4_q4")) as host:
        c, n = host.cfg, host.n_ctx
        kvd = c.n_head_kv * c.head_dim
        rng = np.random.default_rng(21)
        rows = [(rng.standard_normal((n, kvd), dtype=np.float32), rng.standard_normal((n, kvd), dtype=np.float32))
                for _ in range(c.n_layer)]
        with fw_cpu.OracleModel(host) as om:
            for layer, (k, v) in enumerate(rows):
                om.set_kv(layer, 0, k, v)
            ref = om.forward(17, 40)
            t, exp = fw_cpu.argmax(ref), []
            nxt = t
            for i in range(6):
                t = fw_cpu.argmax(om.forward(int(t), 41 + i))
                exp.append(t)
        ctx = per_phase_kernels() if not persistent else open(os.devnull)
        with ctx, fwgpu.GpuModel(host) as gm:
            assert gm.persistent == persistent
            for layer, (k, v) in enumerate(rows):
                gm.kv_write(layer, 0, k, v)
            close(gm.forward(17, 40), ref, "logits at position 40")
            assert np.array_equal(gm.decode_from(nxt, 41, 6), exp)
            gm.decode_from(nxt, 41, 3, copy_out=False)
            assert np.array_equal(gm.decode(3), exp[3:])


def test_persistent_abort_resets_tagged_state(monkeypatch):
    """A persistent launch that starts with the error word set (failure injected
    from the host with FORWORD_GPU_ABORT_LAUNCH): every bounded wait in it takes
    its exit, the call reports the failure, and the next launch, after the epoch
    and every tagged buffer (x, q, the K/V row, the attention partials and
    output) went back to zero, matches the oracle."""
    monkeypatch.setenv("FORWORD_GPU_ABORT_LAUNCH", "2")
    with fwgpu.HostModel(synth=spec_of("hd64_g4_q4")) as host, fwgpu.GpuModel(host) as gm, \
            fw_cpu.OracleModel(host) as om:
        assert gm.persistent
        prompt = np.array([5, 6, 7, 8], np.uint32)
        toks = gm.generate_greedy(prompt, 4)                           # launch 1: positions 0..6
        pos = len(prompt) + 3
        with pytest.raises(fwgpu.ForwordError, match="timed out"):
            gm.decode_from(int(toks[-1]), pos, 3)                      # launch 2: aborted
        got = gm.decode_from(int(toks[-1]), pos, 5)                    # launch 3
        for p, t in enumerate(list(prompt) + list(toks)):
            logits = om.forward(int(t), p)
        exp = []
        for p in range(pos + 1, pos + 6):
            exp.append(fw_cpu.argmax(logits))
            logits = om.forward(exp[-1], p)
        assert list(got) == exp, (got, exp)
