"""Batched prefill (forword_gpu_prefill): the prompt in one pass per layer must
give what forword.c's token-by-token prefill gives (main.c:145-151, one
transformer_forward per prompt token): the last token's logits within max-abs
2e-3 / rel 1e-3 of the reference's (golden fixtures) and the oracle's, the KV
rows within the same tolerance of the token-by-token GPU path, and an
identical greedy continuation.  The linears are GEMMs that sum in another
order, so equality is within the tolerance, not bitwise."""
import numpy as np
import pytest

import fw_cpu
import fwgpu
import golden_specs as gs
from conftest import gold_model

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-3, 1e-3


def close(got, exp, what):
    err = np.abs(got.astype(np.float64) - exp.astype(np.float64))
    bad = ~(err <= ATOL + RTOL * np.abs(exp))                  # NaN counts as out of tolerance
    assert not bad.any(), f"{what}: {bad.sum()} elements out of tolerance, max err {err.max():.3g}"
    return float(err.max())


@pytest.fixture(scope="module", params=list(gs.MODELS))
def fixture_model(request):
    name = request.param
    m = gs.MODELS[name]
    host = fwgpu.HostModel(synth=m["spec"](), max_ctx=m["max_ctx"])
    yield name, host, gold_model(name)
    host.close()


def test_prefill_logits_match_reference(fixture_model):
    name, host, gold = fixture_model
    prompt = gs.prompt(name)
    f = len(prompt) - 1
    with fwgpu.GpuModel(host) as gm:
        lg = gm.prefill(prompt)
    err = close(lg, gold[f"logits_{f}"], f"{name} prefill logits")
    assert fw_cpu.argmax(lg) == int(gold["stats"][f, 0])
    print(f"{name}: max logit err {err:.3g}")


def test_greedy_after_prefill_identical_to_reference(fixture_model):
    name, host, gold = fixture_model
    prompt = gs.prompt(name)
    n_gen = gs.MODELS[name]["n_gen"]
    with fwgpu.GpuModel(host) as gm:
        got = gm.generate_greedy_batched(prompt, n_gen)
    assert np.array_equal(got, gold["tokens"][len(prompt):]), (got, gold["tokens"][len(prompt):])


def test_prefill_kv_rows_match_token_by_token():
    m = gs.MODELS["gqa"]
    prompt = gs.prompt("gqa")
    with fwgpu.HostModel(synth=m["spec"]()) as host:
        with fwgpu.GpuModel(host) as gm:
            for p, t in enumerate(prompt):
                gm.forward(int(t), p)
            ref = [gm.kv_read(l, 0, len(prompt)) for l in range(host.cfg.n_layer)]
        with fwgpu.GpuModel(host) as gm:
            gm.prefill(prompt)
            for l in range(host.cfg.n_layer):
                k, v = gm.kv_read(l, 0, len(prompt))
                close(k, ref[l][0], f"K rows of layer {l}")
                close(v, ref[l][1], f"V rows of layer {l}")


def q4_spec():
    # head_dim 128, GQA group 4, Q4_0 linears (the 8B layout at a small size)
    return fwgpu.spec(512, 1024, 2, 4, 1, 2000, 640, 500000.0, linear_type=gs.Q4, seed=404)


def test_prefill_q4_0_against_oracle():
    prompt = np.random.default_rng(9).integers(3, 2000, 40).astype(np.uint32)
    with fwgpu.HostModel(synth=q4_spec()) as host, fw_cpu.OracleModel(host) as om:
        for p, t in enumerate(prompt[:-1]):
            om.forward(int(t), p)
        exp = om.forward(int(prompt[-1]), len(prompt) - 1)
        with fwgpu.GpuModel(host) as gm:
            got = gm.prefill(prompt)
        close(got, exp, "Q4_0 prefill logits vs oracle")
        assert fw_cpu.argmax(got) == fw_cpu.argmax(exp)


def test_prefill_in_passes_and_continued():
    """600 tokens: two passes inside one call (512 + 88) and the same prompt split
    over two calls (pos0 > 0) agree with the token-by-token GPU path."""
    prompt = np.random.default_rng(10).integers(3, 2000, 600).astype(np.uint32)
    with fwgpu.HostModel(synth=q4_spec()) as host:
        with fwgpu.GpuModel(host) as gm:
            for p, t in enumerate(prompt[:-1]):
                gm.forward_argmax(int(t), p)
            exp = gm.forward(int(prompt[-1]), len(prompt) - 1)
        with fwgpu.GpuModel(host) as gm:
            close(gm.prefill(prompt), exp, "600-token prefill")
        with fwgpu.GpuModel(host) as gm:
            gm.prefill(prompt[:300])
            close(gm.prefill(prompt[300:], 300), exp, "prefill continued at position 300")


def test_prefill_errors():
    m = gs.MODELS["gqa"]
    with fwgpu.HostModel(synth=m["spec"]()) as host, fwgpu.GpuModel(host) as gm:
        with pytest.raises(fwgpu.ForwordError):
            gm.prefill([1] * (host.n_ctx + 1))
        assert "exceed" in fwgpu.last_error()
        with pytest.raises(fwgpu.ForwordError):
            gm.prefill([host.cfg.n_vocab])
        assert "out of range" in fwgpu.last_error()
        gm.prefill([5, 6, 7])                                          # still usable after errors
