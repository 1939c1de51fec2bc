import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device and the built HIP library")


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle

    oracle.load()
    return oracle


@pytest.fixture(scope="session")
def hip():
    """The HIP backend; GPU tests fail loudly (not skip) if it cannot run."""
    import fastembedr_amd as fe
    from fastembedr_amd import _lib

    _lib.load()
    if not fe.available():
        raise RuntimeError("no gfx950 HIP device visible to the HIP backend")
    return fe
