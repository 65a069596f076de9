import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "llm-sys-project_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def amd():
    """The HIP library; GPU tests fail loudly if it is not built."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this container")
    import amdmoe
    amdmoe.load()
    return amdmoe
