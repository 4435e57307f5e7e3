"""Shared test setup: the `gpu` marker, repo-root imports, fixtures."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs on the GPU box")
    config.addinivalue_line("markers", "slow: long CPU sweep, opt-in with NOVAQ_EXHAUSTIVE=1")


def pytest_collection_modifyitems(config, items):
    have_gpu = False
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:
        pass
    for item in items:
        if "gpu" in item.keywords and not have_gpu:
            item.add_marker(pytest.mark.skip(reason="no HIP device in this container"))
        if "slow" in item.keywords and os.environ.get("NOVAQ_EXHAUSTIVE") != "1":
            item.add_marker(pytest.mark.skip(reason="set NOVAQ_EXHAUSTIVE=1"))


@pytest.fixture(scope="session")
def golden():
    d = os.path.join(ROOT, "tests", "golden")
    return {
        "casts": dict(np.load(os.path.join(d, "cast_vectors.npz"))),
        "products": dict(np.load(os.path.join(d, "product_vectors.npz"))),
    }
