"""Shared test setup: import paths, the `gpu` marker, fixtures.

`-m "not gpu"` runs the oracle, ABI and host-logic tests (no GPU needed);
`-m gpu` runs the parity tests of the HIP kernels against the oracle.
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "qwen38-27b-exl3-rdna4_amd")
for p in (PKG, os.path.join(REPO, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(REPO, "tests", "golden", "exl3_golden.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def golden():
    import json
    import numpy as np
    g = np.load(GOLDEN, allow_pickle=False)
    with open(os.path.splitext(GOLDEN)[0] + ".json") as f:
        meta = json.load(f)
    return g, meta
