"""Shared test setup: import paths, the `gpu` marker, and session fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "dflash-swift_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle.qmm_oracle import COracle
    return COracle()


@pytest.fixture(scope="session")
def ctx():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import dflash_qmm
    c = dflash_qmm.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()
