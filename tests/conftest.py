import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, TESTS):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(TESTS, "golden", "attention_golden.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


def load_golden():
    """{case name: {array name: array}} from tests/golden/attention_golden.npz."""
    data = np.load(GOLDEN, allow_pickle=False)
    cases: dict[str, dict[str, np.ndarray]] = {}
    for key in data.files:
        name, field = key.split("/")
        cases.setdefault(name, {})[field] = data[key]
    return cases


@pytest.fixture(scope="session")
def golden():
    return load_golden()
