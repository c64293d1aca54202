import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")


def pytest_collection_modifyitems(config, items):
    # GPU tests fail loudly when selected without a device; they are never
    # silently routed to a CPU path.
    pass


@pytest.fixture(scope="session")
def golden():
    import json
    import numpy as np
    path = os.path.join(ROOT, "tests", "golden", "fit_state_vectors.npz")
    data = np.load(path)
    meta = json.loads(bytes(data["meta"]).decode())
    return data, meta
