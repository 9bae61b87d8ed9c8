import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "base-mlx_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

# tests/test_sanitizers.py runs CPU tests in child processes against the
# AddressSanitizer / UndefinedBehaviorSanitizer builds: "lib" swaps in the
# library's, "oracle" the oracle's (one sanitizer runtime per process).
_SAN = os.environ.get("BMX_TEST_SANITIZED", "")
if _SAN == "lib":
    import bmx._lib as _bmx_lib

    _bmx_lib.LIB_PATH = os.path.join(ROOT, "base-mlx_amd", "lib", "libbmx_san.so")
elif _SAN == "oracle":
    import oracle as _oracle

    _oracle.LIB_PATH = os.path.join(ROOT, "oracle", "_build", "liboracle_san.so")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")
    config.addinivalue_line("markers", "slow: long CPU test")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gpu():
    """The HIP library on cuda:0; fails loudly if it is missing."""
    import torch

    import bmx

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but torch.cuda.is_available() is False")
    bmx.load()
    return bmx
