import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


def _gpu_available() -> bool:
    try:
        from tatara_amd import _lib
        import ctypes as C

        lib = _lib.load()
        n = C.c_int32(0)
        return lib.tatara_device_count(C.byref(n)) == 0 and n.value > 0
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """The HIP library, after checking that a GPU is visible.

    A GPU test run on a machine without a GPU fails (it is not skipped), so a
    silent CPU pass is impossible: the product has no CPU path.
    """
    from tatara_amd import _lib

    lib = _lib.load()
    assert _gpu_available(), "no GPU visible to the HIP library"
    return lib


@pytest.fixture(scope="session")
def oracle():
    from oracle import ffi

    ffi.lib()
    return ffi
