import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "ferrum-gpu_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def orc():
    import oracle

    if not os.path.exists(oracle.LIB_PATH):
        import subprocess

        subprocess.run(["make", "-C", os.path.join(REPO, "oracle")], check=True)
    oracle.lib()
    return oracle
