import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libytm.so on the GPU)")


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle as o

    o.load()
    return o
