import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden")
for p in (os.path.join(ROOT, "forword.c_amd"), os.path.join(ROOT, "oracle"), GOLD):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")
    config.addinivalue_line("markers", "slow: large-shape test (minutes of CPU oracle time)")


@pytest.fixture(scope="session")
def manifest():
    with open(os.path.join(GOLD, "manifest.json")) as f:
        return json.load(f)


def load_npz(name):
    with np.load(os.path.join(GOLD, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def gold_ops():
    return load_npz("ops.npz")


@pytest.fixture(scope="session")
def gold_matvec():
    return load_npz("matvec.npz")


@pytest.fixture(scope="session")
def gold_dequant():
    return load_npz("dequant.npz")


@pytest.fixture(scope="session")
def gold_kquant():
    return load_npz("kquant.npz")


def gold_model(name):
    return load_npz(f"model_{name}.npz")


def check_logit_stats(lg, row, f, atol=2e-3, rtol=1e-3, strict=True):
    """A reference-written statistics row of one forward (ref_driver's gen mode:
    argmax, max logit, largest logit at another index, their difference, double
    sum of all logits) against logits `lg`, each within what the per-logit bar
    |got - exp| <= atol + rtol |exp| allows.  With strict=False (a forward whose
    argmax feeds nothing, e.g. inside a prompt) another argmax is accepted when
    the expected top two are closer than that bar."""
    best = int(np.argmax(lg))
    tol = lambda x: atol + rtol * abs(x)
    tie = best != int(row[0])
    if tie:
        assert not strict, f"greedy choice differs at forward {f}"
        assert row[3] <= tol(row[1]) + tol(row[2]), f"argmax differs at forward {f} beyond a near-tie"
    rest = lg.astype(np.float64)
    rest[best] = -np.inf
    second = float(rest.max())
    k = 2 if tie else 1
    assert abs(float(lg[best]) - row[1]) <= k * tol(row[1]), f"max logit at forward {f}: {lg[best]} vs {row[1]}"
    assert abs(second - row[2]) <= k * tol(row[2]), f"runner-up at forward {f}: {second} vs {row[2]}"
    assert abs((float(lg[best]) - second) - row[3]) <= k * (tol(row[1]) + tol(row[2])), f"margin at forward {f}"
    sum_tol = lg.size * atol + rtol * float(np.abs(lg.astype(np.float64)).sum())
    got_sum = float(np.sum(lg, dtype=np.float64))
    assert abs(got_sum - row[4]) <= sum_tol, f"logit sum at forward {f}: {got_sum} vs {row[4]}"


class kernel_choice:
    """FORWORD_GPU_MEGAKERNEL=0 selects the per-phase kernels for handles
    opened inside the block; otherwise the persistent step kernel runs where
    the model allows it."""

    def __init__(self, persistent):
        self.persistent = persistent

    def __enter__(self):
        if not self.persistent:
            os.environ["FORWORD_GPU_MEGAKERNEL"] = "0"

    def __exit__(self, *a):
        os.environ.pop("FORWORD_GPU_MEGAKERNEL", None)
