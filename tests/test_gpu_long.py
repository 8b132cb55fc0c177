"""Parity at the measured workloads' full shapes (transformer.c:149-326 with
attention.c:142-164 over kv_cache.h:45-51) on both step implementations, against the oracle:

- long context: the 8B attention shape (32 query / 8 KV heads of 128) with a
  KV cache of 32768 positions of N(0,1) rows written through kv_write, decoded
  at positions where split-K attention runs 9 splits per KV head (520), where
  the split count reaches its cap (2100) and at the cache's far end (32768);
- the 70B shape (dim 8192, 80 layers, 64/8 heads, ffn 28672): 4 prompt and
  4 greedy tokens.

Bar: logits within max-abs 2e-3 / rel 1e-3, identical greedy tokens."""
import os

import numpy as np
import pytest

import fw_cpu
import fwgpu
from conftest import kernel_choice

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-3, 1e-3


def close(got, exp, what):
    err = np.abs(got.astype(np.float64) - exp.astype(np.float64))
    bad = ~(err <= ATOL + RTOL * np.abs(exp))                  # NaN counts as out of tolerance
    assert not bad.any(), f"{what}: {bad.sum()} elements out of tolerance, max err {err.max():.3g}"
    return float(err.max())


def say(msg):
    print(msg, flush=True)


# ── long context ──────────────────────────────────────────────────────────────

LC_CACHE, LC_POSITIONS, LC_STEPS = 32768, (520, 2100, 32768), 4


def lc_spec():
    """8B attention shape, two layers, small FFN and vocabulary, room for 32768 + 8 positions."""
    return fwgpu.spec(4096, 1024, 2, 32, 8, 1000, LC_CACHE + 72, 500000.0, linear_type=fwgpu.GGML_Q4_0,
                      embd_type=fwgpu.GGML_Q8_0, output_type=fwgpu.GGML_Q8_0, seed=32)


def lc_rows(layer):
    rng = np.random.default_rng(100 + layer)
    k = rng.standard_normal((LC_CACHE, 1024), dtype=np.float32)
    v = rng.standard_normal((LC_CACHE, 1024), dtype=np.float32)
    return k, v


@pytest.fixture(scope="module")
def lc_model():
    """The host model and the oracle's logits / greedy tokens for each probed position."""
    fw_cpu.set_threads(16)
    host = fwgpu.HostModel(synth=lc_spec(), max_ctx=LC_CACHE + 72)
    assert host.n_ctx == LC_CACHE + 72
    exp = {}
    with fw_cpu.OracleModel(host) as om:
        for layer in range(host.cfg.n_layer):
            k, v = lc_rows(layer)
            om.set_kv(layer, 0, k, v)
        for p in LC_POSITIONS:
            tok = 11 + p % 997
            lg = om.forward(tok, p)
            nxt, toks = fw_cpu.argmax(lg), []
            t = nxt
            for i in range(LC_STEPS):
                t = fw_cpu.argmax(om.forward(int(t), p + 1 + i))
                toks.append(t)
            exp[p] = (tok, lg, nxt, np.array(toks, np.uint32))
            say(f"oracle at position {p}: next {nxt}, greedy {toks}")
    yield host, exp
    host.close()


@pytest.mark.slow
@pytest.mark.parametrize("persistent", [True, False], ids=["persistent", "per_phase"])
def test_long_context_decode_matches_oracle(lc_model, persistent):
    host, exp = lc_model
    with kernel_choice(persistent), fwgpu.GpuModel(host) as gm:
        assert gm.persistent == persistent
        for layer in range(host.cfg.n_layer):
            k, v = lc_rows(layer)
            gm.kv_write(layer, 0, k, v)
        k2, v2 = gm.kv_read(1, LC_CACHE - 3, 3)
        assert np.array_equal(k2, lc_rows(1)[0][-3:]) and np.array_equal(v2, lc_rows(1)[1][-3:])
        for p in LC_POSITIONS:
            tok, lg_ref, nxt, toks = exp[p]
            lg = gm.forward(tok, p)
            e = close(lg, lg_ref, f"logits at position {p}")
            assert fw_cpu.argmax(lg) == nxt
            got = gm.decode_from(nxt, p + 1, LC_STEPS)
            assert np.array_equal(got, toks), (p, got, toks)
            say(f"position {p}: max logit err {e:.3g}, greedy {list(got)}")


# ── 70B shape ─────────────────────────────────────────────────────────────────

@pytest.mark.slow
def test_70b_shape_prompt_and_greedy_match_oracle():
    """Llama-3-70B shape, Q4_0 linears and Q8_0 embedding / output: 4 prompt
    tokens + 4 greedy tokens on the persistent kernel, logits of the last
    forward, against the row-parallel oracle."""
    fw_cpu.set_threads(16)
    prompt = np.random.default_rng(70).integers(3, 128256, 4).astype(np.uint32)
    say("70B: writing the synthetic model")
    os.environ["FW_SYNTH_PROGRESS"] = "1"                   # ~42 GB of weights: report each tenth
    try:
        host = fwgpu.HostModel(synth=fwgpu.spec_70b(n_ctx=16))
    finally:
        os.environ.pop("FW_SYNTH_PROGRESS", None)
    with host:
        say("70B: decoding on the GPU")
        with fwgpu.GpuModel(host) as gm:
            assert gm.persistent
            got = gm.generate_greedy(prompt, 4)
            lg = gm.forward(int(got[-1]), len(prompt) + 3)
        say(f"70B: GPU tokens {list(got)}; running the oracle")
        with fw_cpu.OracleModel(host) as om:
            exp = om.generate_greedy(prompt, 4)
            ref = om.forward(int(exp[-1]), len(prompt) + 3)
    assert np.array_equal(got, exp), (got, exp)
    say(f"70B: max logit err {close(lg, ref, '70B logits'):.3g}")
