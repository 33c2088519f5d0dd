import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("gpt.c_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def oracle():
    import oracle as oracle_mod
    return oracle_mod.Oracle()


@pytest.fixture(scope="session")
def lib():
    import gptc
    return gptc.load()


@pytest.fixture(scope="session")
def rt(lib):
    """GPU runtime (device 0, library stream) initialised once per session."""
    import gptc
    r = gptc.Runtime(lib)
    r.init()
    return r
