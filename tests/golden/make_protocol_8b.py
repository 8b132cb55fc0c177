"""Writes tests/golden/protocol_8b.npz: the oracle's run of the Llama-3-8B-shape
Q4_0 protocol (512 random prompt tokens, then 256 greedy tokens, main.c:145-217
with temperature 0 and no EOS stop), so the GPU test can compare a full-length
sequence without the oracle's ~20 CPU-minutes at test time.

The model is this repository's seeded writer at the 8B shape (fwgpu.spec_8b,
seed 8); the fixture stores the SHA-256 of its data section so a test on
another machine first proves it regenerated the same weights.  Per forward f
it stores the same five statistics as the reference-written fixtures: argmax,
max logit, largest logit at another index, their difference and the sum of all
logits in double precision.

    python tests/golden/make_protocol_8b.py [threads]
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
GOLD = os.path.join(ROOT, "tests", "golden")
for p in (os.path.join(ROOT, "forword.c_amd"), os.path.join(ROOT, "oracle")):
    sys.path.insert(0, p)
import fw_cpu  # noqa: E402
import fwgpu  # noqa: E402

N_PROMPT, N_GEN, PROMPT_SEED = 512, 256, 512


def protocol_prompt(n_vocab: int) -> np.ndarray:
    return np.random.default_rng(PROMPT_SEED).integers(3, n_vocab, N_PROMPT).astype(np.uint32)


def data_sha256(host: "fwgpu.HostModel") -> str:
    buf = (C.c_uint8 * host.data_size).from_address(host.data)
    return hashlib.sha256(memoryview(buf)).hexdigest()


def stats_row(lg: np.ndarray) -> list:
    best = int(fw_cpu.argmax(lg))
    rest = lg.copy()
    rest[best] = -np.inf
    second = float(rest.max())
    return [best, float(lg[best]), second, float(lg[best]) - second, float(np.sum(lg, dtype=np.float64))]


def main():
    threads = int(sys.argv[1]) if len(sys.argv) > 1 else 8
    fw_cpu.set_threads(threads)
    t0 = time.time()
    with fwgpu.HostModel(synth=fwgpu.spec_8b(n_ctx=N_PROMPT + N_GEN)) as host:
        digest = data_sha256(host)
        prompt = protocol_prompt(host.cfg.n_vocab)
        toks = list(prompt)
        stats = []
        with fw_cpu.OracleModel(host) as om:
            for f in range(N_PROMPT + N_GEN - 1):
                lg = om.forward(int(toks[f]), f)
                stats.append(stats_row(lg))
                if f + 1 >= N_PROMPT:
                    toks.append(stats[-1][0])
                if f % 64 == 0:
                    print(f"forward {f} ({time.time() - t0:.0f} s)", flush=True)
    np.savez_compressed(os.path.join(GOLD, "protocol_8b.npz"), tokens=np.array(toks, np.uint32),
                        stats=np.array(stats, np.float64), data_sha256=np.array(digest))
    print(f"done in {time.time() - t0:.0f} s; generated {toks[N_PROMPT:N_PROMPT + 8]}...")


if __name__ == "__main__":
    main()
