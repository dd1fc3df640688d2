import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on cuda:0)")


def _has_gpu() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    if not _has_gpu():
        pytest.skip("no GPU visible")
    import torch

    torch.cuda.set_device(0)
    import lc_parallel_primitive_amd as lcpp

    lcpp.lib()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")


def golden(name, dtype):
    import numpy as np

    return np.fromfile(os.path.join(GOLDEN, name), dtype=dtype)


def log(msg: str) -> None:
    """Name the case before each GPU step (flushed), so a crash log shows it."""
    print(f"[case] {msg}", flush=True)
