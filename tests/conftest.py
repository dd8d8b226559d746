import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# a crash inside the native library prints its native stack (host.cpp)
os.environ.setdefault("LLMHIP_CRASH_TRACE", "1")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libllmhip.so on cuda:0)")


@pytest.fixture(scope="session")
def gpu():
    """The GPU tests run only where a GPU exists; there they must not be
    skipped.  The process loads one HIP runtime, the one libllmhip.so links
    (torch, which bundles another, is not imported by these tests)."""
    from llm_amd import _lib
    _lib.lib()  # raises if libllmhip.so was not built
    if _lib.device_count() < 1:
        pytest.fail("a gpu-marked test ran without a GPU (run `pytest -m 'not gpu'` on CPU machines)")
    return 0


@pytest.fixture(scope="session")
def oracle():
    from oracle import cpuref
    cpuref.lib()
    return cpuref
