import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libtensor_ops_hip.so on the GPU)")
    config.addinivalue_line("markers", "slow: exhaustive sweeps (tens of seconds)")


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle import oracle as O
    return O.oracle()


@pytest.fixture(scope="session")
def hip():
    """The HIP library driven through its C ABI; GPU tests fail loudly without it."""
    # torch bundles its own libamdhip64.so.7.  Whichever copy is loaded first
    # serves the whole process, and torch cannot initialise on a runtime that
    # another library loaded before it.  Initialise torch first (as bench.py
    # does) so the tests that use torch for device plumbing share its runtime.
    try:
        import torch
        torch.cuda.init()
    except Exception:
        pass
    from tests.helpers import HipLib
    lib = HipLib()
    if lib.device_count() == 0:
        pytest.fail("libtensor_ops_hip.so reports no GPU (these tests need an MI355X)")
    return lib
