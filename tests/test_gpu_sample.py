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


def test_sampled_generation_nucleus_too_large():
    # tiny model: 32000 near-uniform logits, top_p 0.99 needs ~31700 tokens
    m = gs.MODELS["tiny"]
    with fwgpu.HostModel(synth=m["spec"]()) as host, fwgpu.GpuModel(host) as gm:
        with pytest.raises(fwgpu.ForwordError):
            gm.generate(gs.prompt("tiny"), 4, 1.0, 0.99, 1.0, 9)
        assert "nucleus" in fwgpu.last_error()
        gm.generate(gs.prompt("tiny"), 4, 0.0, 0.9, 1.1, 9)          # still usable
