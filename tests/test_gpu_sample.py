"""Device-resident sampled generation (forword_gpu_generate) against the oracle's
restatement of the CLI loop (main.c:145-217 with sampler.c:12-101), itself
pinned to the compiled reference's sampler decisions (tests/test_oracle.py):
identical token sequences for greedy-with-penalty and top-p settings."""
import numpy as np
import pytest

import fw_cpu
import fwgpu
import golden_specs as gs

pytestmark = pytest.mark.gpu

SETTINGS = [(0.0, 0.9, 1.3, 1), (0.8, 0.9, 1.1, 12345), (1.0, 0.95, 1.0, 77), (1.5, 0.5, 1.2, 2 ** 40 + 3),
            (0.6, 0.3, 1.05, 0), (0.9, 0.0, 1.1, 31)]          # top_p 0: the nucleus is the top token


@pytest.mark.parametrize("name", ["gqa", "q5", "qwen2", "phi2", "gpt2"])   # persistent and per-phase steps
def test_sampled_generation_matches_oracle(name):
    m = gs.MODELS[name]
    prompt = gs.prompt(name)
    with fwgpu.HostModel(synth=m["spec"](), max_ctx=m["max_ctx"]) as host, fw_cpu.OracleModel(host) as om:
        with fwgpu.GpuModel(host) as gm:
            for (temp, top_p, pen, seed) in SETTINGS:
                exp = om.generate_sampled(prompt, 20, temp, top_p, pen, seed)
                got = gm.generate(prompt, 20, temp, top_p, pen, seed)
                assert np.array_equal(got, exp), (temp, top_p, pen, seed, got, exp)


def test_sampled_generation_greedy_equals_greedy_loop():
    m = gs.MODELS["gqa"]
    prompt = gs.prompt("gqa")
    with fwgpu.HostModel(synth=m["spec"]()) as host, fwgpu.GpuModel(host) as gm:
        assert np.array_equal(gm.generate(prompt, 16, 0.0, 0.9, 1.0, 5), gm.generate_greedy(prompt, 16))


def test_sampled_generation_repeats_bitwise():
    # the same seed gives the same tokens: no order-dependent accumulation decides a draw
    m = gs.MODELS["gqa"]
    prompt = gs.prompt("gqa")
    with fwgpu.HostModel(synth=m["spec"]()) as host, fwgpu.GpuModel(host) as gm:
        runs = [gm.generate(prompt, 24, 1.2, 0.9, 1.1, 4242) for _ in range(3)]
        assert all(np.array_equal(runs[0], r) for r in runs[1:])


def test_sampled_generation_large_nucleus_matches_oracle():
    # tiny model: 32000 near-uniform logits, top_p 0.99 needs ~31700 candidates,
    # more than the LDS sort holds: the global-buffer sort takes them
    m = gs.MODELS["tiny"]
    prompt = gs.prompt("tiny")
    with fwgpu.HostModel(synth=m["spec"]()) as host, fw_cpu.OracleModel(host) as om:
        exp = om.generate_sampled(prompt, 4, 1.0, 0.99, 1.0, 9)
        with fwgpu.GpuModel(host) as gm:
            got = gm.generate(prompt, 4, 1.0, 0.99, 1.0, 9)
            again = gm.generate(prompt, 4, 1.0, 0.99, 1.0, 9)
            gm.generate(prompt, 4, 0.0, 0.9, 1.1, 9)                  # the greedy path after it
    assert np.array_equal(got, exp), (got, exp)
    assert np.array_equal(got, again)


def test_sampled_generation_full_vocabulary_nucleus():
    # a 128256-token vocabulary (Llama 3) at temperature 1.5, top_p 0.95: the
    # nucleus holds most of the vocabulary
    sp = fwgpu.spec(256, 512, 2, 8, 2, 128256, 64, 500000.0, seed=128)
    prompt = np.random.default_rng(128).integers(3, 128256, 6).astype(np.uint32)
    with fwgpu.HostModel(synth=sp) as host, fw_cpu.OracleModel(host) as om:
        exp = om.generate_sampled(prompt, 6, 1.5, 0.95, 1.0, 1234)
        with fwgpu.GpuModel(host) as gm:
            got = gm.generate(prompt, 6, 1.5, 0.95, 1.0, 1234)
            again = gm.generate(prompt, 6, 1.5, 0.95, 1.0, 1234)
    assert np.array_equal(got, exp), (got, exp)
    assert np.array_equal(got, again)
