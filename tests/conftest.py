import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libsiphon_hip.so)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import siq
    return siq.Oracle()


@pytest.fixture(scope="session")
def ref():
    """The compiled reference (oracle/_ref), or skip when it was not built."""
    from oracle import siq
    r = siq.Reference.load()
    if r is None:
        pytest.skip("oracle/_ref not built (needs /root/reference at build time)")
    return r


@pytest.fixture(scope="session")
def emu():
    from tests import emu_py
    return emu_py.Emulator()


@pytest.fixture(scope="session")
def dev():
    import siphon_amd
    d = siphon_amd.Device(0)
    yield d
    d.close()


@pytest.fixture
def option(dev):
    """Set tuning options on the session device for one test: option(name,
    value); every option set is restored to its built-in rule afterwards."""
    touched = []

    def set_(name, value):
        dev.set_option(name, value)
        touched.append(name)

    yield set_
    for name in touched:
        dev.set_option(name, -1)
