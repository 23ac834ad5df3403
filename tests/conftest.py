import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "moe-offload_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI library)")


def _banner(item):
    # Name the case before every GPU test so a run that takes the machine down still says which.
    if item.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-test] {item.nodeid}", flush=True)


def pytest_runtest_setup(item):
    _banner(item)


@pytest.fixture(scope="session")
def golden_moe():
    import numpy as np
    return dict(np.load(GOLDEN / "moe_fixture.npz"))


@pytest.fixture(scope="session")
def lru_traces():
    import json
    return json.loads((GOLDEN / "lru_traces.json").read_text())
