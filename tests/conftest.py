"""Test configuration: the `gpu` marker, import paths and shared fixtures.

CPU tests (`-m "not gpu"`) pin the oracle (oracle/) against the reference
anchors, float64 truths and exact corners, and check the C ABI library
loads and exports its symbols. GPU tests (`-m gpu`) are the parity tests
proper: the HIP library through its C ABI against the oracle on the same
seeded inputs.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "apus-qwen3.6-35b-a3b_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle.Oracle()


@pytest.fixture(scope="session")
def ref():
    import oracle
    if not oracle.Reference.available():
        pytest.skip("reference anchors not built (oracle/_ref needs /root/reference)")
    return oracle.Reference()


@pytest.fixture(scope="session")
def hip():
    """The HIP library; fails loudly (never skips) when it cannot run."""
    import apus_hip
    apus_hip.init(0)
    return apus_hip


@pytest.fixture
def rng(request):
    seed = abs(hash(request.node.name)) % (2**32)
    return np.random.default_rng(seed)
