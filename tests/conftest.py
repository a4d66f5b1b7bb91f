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


def rel_l2(got, ref):
    """Relative L2 error per output vector (rows of a 2-D array), as the parity contract."""
    import numpy as np
    got = np.atleast_2d(np.asarray(got, np.float64))
    ref = np.atleast_2d(np.asarray(ref, np.float64))
    num = np.linalg.norm(got - ref, axis=-1)
    den = np.linalg.norm(ref, axis=-1)
    return np.where(den > 0, num / np.maximum(den, 1e-300), num)


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a GPU")
    import kata_amd
    kata_amd.lib()          # loud failure if the HIP library is missing
    return torch.device("cuda:0")
