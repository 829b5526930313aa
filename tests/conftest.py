import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def q():
    """The HIP backend package (raises if libq35hip.so is not built).

    With Q35_EMULATION_LIB set (tests/emu, never on a GPU run) the same tests
    drive the AddressSanitizer host build of the kernels instead."""
    emu = os.environ.get("Q35_EMULATION_LIB")
    if emu:
        from tests.emu.twin import load_twin
        return load_twin(emu)
    import __graft_entry__ as entry
    return entry.load()


@pytest.fixture(scope="session")
def ctx(q):
    c = q.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="session")
def orc():
    from oracle import q35_oracle
    return q35_oracle
