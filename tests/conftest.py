import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gb300-rl-runtime_amd")
ORACLE = os.path.join(ROOT, "oracle")
for p in (PKG, ORACLE):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


@pytest.fixture(scope="session")
def rl():
    import rlrt
    rlrt.lib()  # raises if the library is not built
    return rlrt


@pytest.fixture(scope="session")
def orc():
    import orc as orc_mod
    return orc_mod


@pytest.fixture(scope="session")
def olib(orc):
    return orc.load_oracle()


@pytest.fixture(scope="session")
def gpu(rl):
    """Opens device 0 through the C ABI. Skips only where no GPU driver exists;
    on a GPU machine any failure to open is an error."""
    if not os.path.exists("/dev/kfd"):
        pytest.skip("no GPU driver (/dev/kfd) on this machine")
    info = rl.open_device(0)
    print(f"\n[gpu] {info.arch.decode()} cu={info.cu_count} hbm={info.hbm_bytes >> 30} GiB", flush=True)
    return info
