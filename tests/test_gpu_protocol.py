"""The Llama-3-8B-shape Q4_0 protocol (main.c:145-217 with temperature 0 and
no EOS stop): 512 random prompt tokens then 256 greedy tokens, token by token
and after the batched prefill, on both step implementations, against the
oracle's run stored in tests/golden/protocol_8b.npz (written by
tests/golden/make_protocol_8b.py; the oracle takes ~20 CPU-minutes for it).
Every one of the 767 forwards is also checked through the logits' argmax, max,
runner-up, margin and sum.  Bar: logits within max-abs 2e-3 / rel 1e-3,
identical greedy tokens."""
import ctypes as C
import hashlib
import os

import numpy as np
import pytest

import fwgpu
from conftest import check_logit_stats, kernel_choice

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_protocol():
    with np.load(os.path.join(GOLD, "protocol_8b.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def protocol_model():
    gold = load_protocol()
    n_prompt = int(gold["tokens"].size - 256)
    with fwgpu.HostModel(synth=fwgpu.spec_8b(n_ctx=gold["tokens"].size)) as host:
        buf = (C.c_uint8 * host.data_size).from_address(host.data)
        assert hashlib.sha256(memoryview(buf)).hexdigest() == str(gold["data_sha256"]), \
            "the synthetic 8B model differs from the one the fixture was written for"
        yield host, gold, n_prompt


@pytest.mark.slow
@pytest.mark.parametrize("persistent", [True, False], ids=["persistent", "per_phase"])
def test_8b_protocol_greedy_identical_to_oracle(protocol_model, persistent):
    host, gold, n_prompt = protocol_model
    prompt, exp = gold["tokens"][:n_prompt], gold["tokens"][n_prompt:]
    with kernel_choice(persistent), fwgpu.GpuModel(host) as gm:
        assert gm.persistent == persistent
        got = gm.generate_greedy(prompt, exp.size)
        assert np.array_equal(got, exp), f"token by token: first difference at {np.argmax(got != exp)}"
        got_b = gm.generate_greedy_batched(prompt, exp.size)
        assert np.array_equal(got_b, exp), f"after prefill: first difference at {np.argmax(got_b != exp)}"


@pytest.mark.slow
def test_8b_protocol_per_forward_statistics(protocol_model):
    """Every one of the 767 forwards: the logits' argmax, max, runner-up, margin
    and sum against the oracle's."""
    host, gold, n_prompt = protocol_model
    toks, stats = gold["tokens"], gold["stats"]
    with fwgpu.GpuModel(host) as gm:
        for f in range(stats.shape[0]):
            check_logit_stats(gm.forward(int(toks[f]), f), stats[f], f, strict=f + 1 >= n_prompt)
