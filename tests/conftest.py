"""Shared pytest setup: import paths and the ``gpu`` marker."""

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (REPO, os.path.join(REPO, "pytorch-engine_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(REPO, "tests", "golden", "ref_vectors.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box only)")


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}
