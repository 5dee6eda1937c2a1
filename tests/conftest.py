"""Shared test setup.

Markers: `gpu` tests need an MI355X (run with `-m gpu`); everything else runs
on a CPU-only host.  The package lives in flash-train_amd/ and the oracle in
oracle/; both are put on sys.path here.
"""

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO, "flash-train_amd")
for p in (PKG_ROOT, REPO):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(REPO, "tests", "golden", "gemm_golden.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    o.build() if not os.path.exists(o.LIB_PATH) else None
    return o
