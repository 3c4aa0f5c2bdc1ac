import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "cis2-lab-archive_amd")
for p in (PKG, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: takes tens of seconds on CPU")


def load_golden(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def model_fixtures():
    return load_golden("model_fixtures.json")


@pytest.fixture(scope="session")
def math_fixture():
    return load_golden("math_chunk_hashes.json")


@pytest.fixture(scope="session")
def rust5():
    return load_golden("rust5_gemv_hashes.json")
