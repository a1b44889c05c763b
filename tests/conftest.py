import contextlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN


@pytest.fixture(scope="session")
def cuda():
    """The GPU device; GPU tests fail (not skip) when no GPU is present."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a ROCm GPU"
    import hrm_moe_amd

    hrm_moe_amd.load_library()
    return torch.device("cuda:0")


@contextlib.contextmanager
def lib_env(**values):
    """Set HRM_MOE_* tuning variables (None = unset), reload the library's configuration, restore both after."""
    from hrm_moe_amd import _lib

    saved = {n: os.environ.get(n) for n in values}
    try:
        for n, v in values.items():
            if v is None:
                os.environ.pop(n, None)
            else:
                os.environ[n] = v
        _lib.reload_config()
        yield
    finally:
        for n, v in saved.items():
            if v is None:
                os.environ.pop(n, None)
            else:
                os.environ[n] = v
        _lib.reload_config()
