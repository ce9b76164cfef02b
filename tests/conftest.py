import os
import sys

import pytest

# torch carries its own HIP runtime (soname libamdhip64.so.7). Imported
# before the backend library is loaded, it serves both, so the test process
# has one runtime; the tests that use torch tensors need that. The reference
# harness tests (test_gpu_vtable.py) run in child processes without torch,
# on the system runtime, as a C consumer of the backend does.
try:
    import torch  # noqa: F401
except ImportError:
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long CPU oracle runs")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    return oracle.lib()
