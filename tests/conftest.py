import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); run with -m gpu")
    config.addinivalue_line("markers", "slow: full-size parity case (seconds of oracle work)")


@pytest.fixture(scope="session")
def c_oracle():
    from oracle import c_oracle as co

    co.build()
    return co


@pytest.fixture
def tune():
    """Sets planner overrides (``capi.TUNE`` knobs) for one test; every knob
    it touched is restored afterwards."""
    from piecewiselinearembeddings_optimized_amd import capi

    prev = {}

    def set_(knob, value):
        old = capi.set_tuning(knob, value)
        prev.setdefault(knob, old)

    yield set_
    for knob, value in prev.items():
        capi.set_tuning(knob, value)
