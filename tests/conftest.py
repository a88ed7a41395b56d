import os
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU check")


def gpu_available() -> bool:
    """A HIP device is visible (hipGetDeviceCount through the HIP runtime)."""
    import ctypes

    try:
        hip = ctypes.CDLL("libamdhip64.so")
    except OSError:
        return False
    count = ctypes.c_int(0)
    return hip.hipGetDeviceCount(ctypes.byref(count)) == 0 and count.value > 0


@pytest.fixture(scope="session")
def oracle():
    from oracle import binding

    binding.load()
    return binding


@pytest.fixture(scope="session")
def require_gpu():
    if not gpu_available():
        pytest.fail("GPU test requested but no HIP device is visible")
    return True


def pytest_collection_modifyitems(config, items):
    # GPU tests run only when selected with -m gpu; they never fall back.
    markexpr = config.getoption("-m") or ""
    if "gpu" in markexpr and "not gpu" not in markexpr:
        return
    skip = pytest.mark.skip(reason="GPU test: run with -m gpu on an MI355X")
    for item in items:
        if "gpu" in item.keywords and os.environ.get("LEO_FORCE_GPU_TESTS") != "1":
            item.add_marker(skip)
