import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 (MI355X) device and the built HIP library")
    config.addinivalue_line("markers", "slow: CPU test taking more than ~20 s")
    config.addinivalue_line("markers", "veryslow: CPU test taking minutes; runs with FMLH_RUN_SLOW=1")


def pytest_collection_modifyitems(config, items):
    if not os.environ.get("FMLH_RUN_SLOW"):
        skip_slow = pytest.mark.skip(reason="takes minutes on the CPU; set FMLH_RUN_SLOW=1 to run")
        for item in items:
            if "veryslow" in item.keywords:
                item.add_marker(skip_slow)
    # A GPU test must never pass silently without the device: it runs only where one is
    # present (/dev/kfd) and then fails loudly if the native library is missing.
    if os.path.exists("/dev/kfd"):
        return
    skip = pytest.mark.skip(reason="no GPU in this environment (/dev/kfd absent)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


GOLDEN = os.path.join(ROOT, "tests", "golden")


def load_golden(name):
    import numpy as np

    path = os.path.join(GOLDEN, f"{name}.npz")
    if not os.path.exists(path):
        pytest.skip(f"golden fixture {name}.npz not generated")
    return dict(np.load(path, allow_pickle=False))


@pytest.fixture(scope="session")
def golden():
    return load_golden
