import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "supra2-img-web_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def dev():
    """The HIP device through the library's own runtime helpers. Fails (does not skip) when no
    device is visible: GPU tests are only collected with -m gpu."""
    from supra_attn.device import Device

    return Device(0)
