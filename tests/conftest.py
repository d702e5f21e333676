import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oxcoder-9b_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device; runs the HIP kernels")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (test infrastructure), built on demand."""
    from oracle import oracle
    if not os.path.exists(os.path.join(ROOT, "oracle", "libkq_oracle.so")):
        oracle.build()
    return oracle


@pytest.fixture(scope="session")
def golden():
    return np.load(os.path.join(GOLDEN, "kindi_cpu.npz"), allow_pickle=False)


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from kq import _lib
    _lib.kq()            # raises if libkq.so is missing: GPU tests never run without it
    return torch.device("cuda:0")
