import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def kernels():
    """The HIP kernel module, enabled (GPU tests only)."""
    from distributedmoellm_amd import kernels as k
    if not k.ENABLED:
        pytest.fail(f"HIP kernels are not available on this GPU machine: {k.WHY_DISABLED}")
    return k
