import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def engine():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import lastengine_amd as le
    return le.Engine()


@pytest.fixture
def fresh_engine():
    """A context of its own, for tests that change launch options (the session engine keeps the
    defaults)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import lastengine_amd as le
    return le.Engine()
