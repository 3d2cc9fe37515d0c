"""Test configuration: the `gpu` marker and the paths of the oracle and the package."""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "inference.rs_amd"):
    p = os.path.join(REPO, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; parity tests through the C ABI")


def pytest_collection_modifyitems(config, items):
    # a GPU test on a box with no GPU is an error, not a skip: the round-end run must not pass on nothing
    pass


@pytest.fixture(scope="session")
def rng_seed():
    return 20261201
