import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qora-tts-12hz-1.7b_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (runs the HIP library)")


@pytest.fixture(scope="session")
def ctx():
    import qtts

    c = qtts.Context(0)
    yield c
    c.close()
