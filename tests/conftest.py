import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "catena-models_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run on the GPU box)")
    config.addinivalue_line("markers", "slow: long-running check")


@pytest.fixture(scope="session")
def oracle():
    import oracle as ox
    ox.build()
    return ox


@pytest.fixture(scope="session")
def known_answers():
    import json
    with open(os.path.join(ROOT, "tests", "golden", "simt_known_answers.json")) as f:
        return json.load(f)
