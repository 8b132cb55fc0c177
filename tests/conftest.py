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
