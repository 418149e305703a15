import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "tests"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def rel_l2(a, b):
    """sqrt(sum (a-b)^2 / sum b^2) in fp64 (the metric of src/tools/dit_test.cpp:11-21)."""
    import numpy as np
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.sqrt(np.sum((a - b) ** 2) / (np.sum(b ** 2) + 1e-30)))


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.set_threads(min(16, os.cpu_count() or 1))
    return oracle
