import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "abyo-speculate_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def _ensure_oracle():
    lib = os.path.join(ROOT, "oracle", "liboracle.so")
    if not os.path.exists(lib):
        import build_oracle
        build_oracle.build()


_ensure_oracle()


@pytest.fixture(scope="session")
def hip():
    """The HIP binding; the library must be built (no fallback)."""
    import speculate_hip
    speculate_hip.load_library()
    return speculate_hip
