import os
import subprocess
import sys

import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
sys.path.insert(0, os.path.join(ROOT, "welvet.cuda_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a visible MI355X (runs the HIP kernels)")


def pytest_sessionstart(session):
    # The oracle is plain C; build it if this checkout has none yet.
    if not os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so")):
        subprocess.check_call(["make", "-s", "-f", os.path.join(ROOT, "oracle", "Makefile"),
                               os.path.join(ROOT, "oracle", "liboracle.so")])
    # The C++ API probe links libwelvet.so (built by __graft_entry__.build).
    probe = os.path.join(ROOT, "tests", "cpp", "libapi_probe.so")
    if not os.path.exists(probe) and os.path.exists(
            os.path.join(ROOT, "welvet.cuda_amd", "libwelvet.so")):
        subprocess.check_call(["make", "-s", "-f", os.path.join(ROOT, "tests", "cpp", "Makefile")])


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib
    return oracle_lib.Oracle()


@pytest.fixture(scope="session")
def gpu():
    """Initialises device 0 through the library; fails loudly if it cannot."""
    import pywelvet as pw
    L = pw.lib()
    pw.check(L.welvet_cuda_init())
    return pw
