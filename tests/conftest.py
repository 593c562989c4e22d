"""Shared fixtures.  CPU tests (-m "not gpu") cover the oracle against golden
vectors and the reference library, the host logic and the C-ABI exports;
GPU tests (-m gpu) are the parity tests proper, calling through the C-ABI."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "mfft-bench_amd"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    from oracle_ctypes import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle_ctypes import load_reference
    r = load_reference()
    if r is None:
        pytest.skip("reference library not built (oracle/_ref)")
    return r


@pytest.fixture(scope="session")
def lib():
    import mfft_ctypes
    return mfft_ctypes.load()


@pytest.fixture(scope="session")
def gpu(lib):
    """The product library on a gfx950 device; fails (never skips) when the
    device or the library is missing, so a GPU run cannot pass vacuously."""
    import mfft_ctypes
    arch = lib.mfh_device_arch().decode()
    assert lib.mfh_device_count() > 0 and arch.startswith("gfx950"), f"no gfx950 device (arch={arch!r})"
    return mfft_ctypes
