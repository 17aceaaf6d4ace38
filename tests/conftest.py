import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "privacy-rag_amd"), os.path.join(ROOT, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def golden_dir():
    return os.path.join(ROOT, "tests", "golden")


@pytest.fixture(scope="session")
def gpu():
    """torch device handle for the -m gpu tests (they need a gfx950 GPU)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    import praghip
    assert praghip.device_count() >= 1, "praghip sees no gfx950 device"
    return torch.device("cuda:0")


def to_dev(a, device="cuda:0"):
    import numpy as np
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint64:
        a = a.view(np.int64)
    return torch.from_numpy(a).to(device)


def from_dev(t):
    import numpy as np
    a = t.detach().cpu().numpy()
    return a.view(np.uint64) if a.dtype == np.int64 else a
