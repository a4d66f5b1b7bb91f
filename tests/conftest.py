import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs on the GPU box")


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    with np.load(os.path.join(ROOT, "tests", "golden", "ptq1_golden.npz")) as z:
        return {k: z[k] for k in z.files}
