import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run on the GPU box)")


@pytest.fixture(scope="session")
def oracle():
    from oracle_lib import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def lib():
    """The MI355X library, initialised on the device.  A GPU test that cannot
    get the device fails: there is no CPU fallback to pass on."""
    import picograd_amd
    L = picograd_amd.load()
    rc = L.pg_amd_init()
    assert rc == 0, f"device init failed: {L.pg_amd_last_error().decode()}"
    return L
