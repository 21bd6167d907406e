"""pytest configuration: the `gpu` marker and shared fixtures.

Tests marked `gpu` need an MI355X; they call the C ABI through
llmpager_amd and check it against the CPU oracle (oracle/), never the other
way round.  Everything else runs on the CPU.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and runs the HIP kernels")
    config.addinivalue_line("markers", "slow: long CPU test, skipped unless LP_SLOW=1")


def pytest_collection_modifyitems(config, items):
    if os.environ.get("LP_SLOW") == "1":
        return
    skip = pytest.mark.skip(reason="slow test; set LP_SLOW=1")
    for it in items:
        if "slow" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def cuda():
    import llmpager_amd as lp
    c = lp.Cuda(0)
    yield c
    c.sync()
    c.close()
