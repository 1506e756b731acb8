import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle.binding import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def gpu():
    """Initialises the HIP library once per session on device 0."""
    import mojostream_amd as ms
    ms.init(0)
    name, ncu, hbm = ms.device_info()
    print(f"\n[gpu] {name} CUs={ncu} HBM={hbm / 2**30:.0f} GiB", flush=True)
    yield ms
    ms.synchronize()
