"""pytest configuration: the `gpu` marker, import paths and the oracle build."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "ltq-research_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")


@pytest.fixture(scope="session")
def oracle():
    from oracle import ref
    ref.lib()
    return ref


@pytest.fixture(scope="session")
def golden_dir():
    return ROOT / "tests" / "golden"
