import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "pto-wsp_amd"), ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built():
    """Build the native library and the oracle only when they are missing."""
    lib = os.path.join(ROOT, "pto-wsp_amd", "pto_wsp", "libptowsp_hip.so")
    orc = os.path.join(ROOT, "oracle", "_build", "libptowsp_cpusim.so")
    if not os.path.exists(lib) or not os.path.exists(orc):
        import __graft_entry__

        __graft_entry__.build()


_ensure_built()


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch.device("cuda:0")
