import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running parity case")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (test infrastructure), built on demand."""
    from oracle import oracle as O

    O.lib()
    return O


@pytest.fixture(scope="session")
def hip():
    """The HIP backend on device 0.  Fails (does not skip) if the library or
    the device is missing: GPU tests must run the native path."""
    import esolearn_amd as E

    E.init(0)
    info = E.HipBackend.device_info()
    print(f"[gpu] {info}", flush=True)
    return E
