"""Model-level parity of the GPU decode path (forword_gpu_forward / greedy loop)
with forword.c's transformer_forward (golden fixtures) and the oracle:
logits and per-layer residual stream within max-abs 2e-3 / rel 1e-3, and an
identical greedy token sequence."""
import os

import numpy as np
import pytest

import fw_cpu
import fwgpu
import golden_specs as gs
from conftest import check_logit_stats, gold_model

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


def test_forward_logits_and_trace_match_reference(fixture_model):
    name, host, gold = fixture_model
    prompt = gs.prompt(name)
    lsteps, tsteps = gs.logit_steps(name), gs.trace_steps(name)
    toks = gold["tokens"]
    errs = []
    with fwgpu.GpuModel(host) as gm:
        for f in range(gs.n_forwards(name)):
            lg = gm.forward(int(toks[f]), f)
            check_logit_stats(lg, gold["stats"][f], f)
            if f in lsteps:
                errs.append(close(lg, gold[f"logits_{f}"], f"{name} logits at forward {f}"))
            if f in tsteps:
                close(gm.layer_trace().reshape(-1), gold[f"trace_{f}"], f"{name} residual stream at forward {f}")
    print(f"{name}: max logit err {max(errs):.3g}")


def test_greedy_tokens_identical_to_reference(fixture_model):
    name, host, gold = fixture_model
    prompt = gs.prompt(name)
    n_gen = gs.MODELS[name]["n_gen"]
    with fwgpu.GpuModel(host) as gm:
        got = gm.generate_greedy(prompt, n_gen)
    assert np.array_equal(got, gold["tokens"][len(prompt):]), (got, gold["tokens"][len(prompt):])


def test_forward_argmax_and_errors():
    m = gs.MODELS["gqa"]
    with fwgpu.HostModel(synth=m["spec"]()) as host, fwgpu.GpuModel(host) as gm, fw_cpu.OracleModel(host) as om:
        nxt = gm.forward_argmax(7, 0)
        assert nxt == fw_cpu.argmax(om.forward(7, 0))
        assert not gm.forward_raw(0, host.n_ctx)                       # transformer.c:156-159
        assert "exceeds" in fwgpu.last_error()
        assert not gm.forward_raw(host.cfg.n_vocab, 0)                 # transformer.c:161-164
        assert "out of range" in fwgpu.last_error()
        with pytest.raises(fwgpu.ForwordError):
            gm.generate_greedy([1] * 10, host.n_ctx)                   # more forwards than the cache
        gm.forward(7, 1)                                               # still usable after errors


def test_kv_write_read_roundtrip_and_attention_over_written_rows():
    m = gs.MODELS["gqa"]
    with fwgpu.HostModel(synth=m["spec"]()) as host, fwgpu.GpuModel(host) as gm, fw_cpu.OracleModel(host) as om:
        c = host.cfg
        kvd = c.n_head_kv * c.head_dim
        rng = np.random.default_rng(5)
        n = 40
        for layer in range(c.n_layer):
            k = rng.standard_normal((n, kvd)).astype(np.float32)
            v = rng.standard_normal((n, kvd)).astype(np.float32)
            gm.kv_write(layer, 0, k, v)
            om.set_kv(layer, 0, k, v)
            k2, v2 = gm.kv_read(layer, 0, n)
            assert np.array_equal(k2, k) and np.array_equal(v2, v)
        close(gm.forward(11, n), om.forward(11, n), "logits after kv_write prefill")
        k_new, _ = gm.kv_read(0, n, 1)
        close(k_new[0], om.kv(0, n)[0], "appended post-RoPE K row")


def test_graph_replays_match_eager():
    """The per-phase kernels' captured step replayed many times, interleaved
    with eager work and synchronisations, gives the same logits as direct
    launches."""
    m = gs.MODELS["gqa"]
    toks = [3, 99, 512, 7, 7, 800, 1, 42]
    os.environ["FORWORD_GPU_MEGAKERNEL"] = "0"
    try:
        with fwgpu.HostModel(synth=m["spec"]()) as host:
            with fwgpu.GpuModel(host) as gm:
                assert not gm.persistent
                graph_logits = [gm.forward(t, i) for i, t in enumerate(toks)]
                replay_tokens = gm.generate_greedy(toks[:3], 6)
            os.environ["FORWORD_GPU_GRAPH"] = "0"
            try:
                with fwgpu.GpuModel(host) as em:
                    eager_logits = [em.forward(t, i) for i, t in enumerate(toks)]
                    eager_tokens = em.generate_greedy(toks[:3], 6)
            finally:
                del os.environ["FORWORD_GPU_GRAPH"]
    finally:
        del os.environ["FORWORD_GPU_MEGAKERNEL"]
    for a, b in zip(graph_logits, eager_logits):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(replay_tokens, eager_tokens)


def test_prefill_then_decode_matches_forward_loop():
    """generate_greedy (device-resident loop) equals host-driven forward+argmax."""
    m = gs.MODELS["tiny"]
    prompt = gs.prompt("tiny")
    with fwgpu.HostModel(synth=m["spec"]()) as host, fwgpu.GpuModel(host) as gm:
        dev = gm.generate_greedy(prompt, 20)
        toks = list(prompt)
        for f in range(len(prompt) + 19):
            nxt = gm.forward_argmax(int(toks[f]), f)
            if f + 1 >= len(prompt):
                toks.append(nxt)
        assert np.array_equal(dev, np.array(toks[len(prompt):], np.uint32))


@pytest.mark.slow
def test_8b_shape_short_decode_vs_oracle():
    """Llama-3-8B shape (Q4_0 linears, Q8_0 embedding/output): 8 prompt tokens and
    8 greedy tokens on the GPU against the oracle run row-parallel on the host."""
    sp = fwgpu.spec_8b(n_ctx=64)
    prompt = np.random.default_rng(8).integers(3, 128256, 8).astype(np.uint32)
    fw_cpu.set_threads(16)
    with fwgpu.HostModel(synth=sp) as host:
        with fwgpu.GpuModel(host) as gm:
            got = gm.generate_greedy(prompt, 8)
            lg = gm.forward(int(got[-1]), len(prompt) + 7)
        with fw_cpu.OracleModel(host) as om:
            exp = om.generate_greedy(prompt, 8)
            ref = om.forward(int(exp[-1]), len(prompt) + 7)
    assert np.array_equal(got, exp), (got, exp)
    close(lg, ref, "8B logits")
