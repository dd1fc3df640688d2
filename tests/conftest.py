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


def special_float_keys(dtype, n: int, seed: int):
    """Float sort keys in which a quarter of the elements are the values a radix
    sort orders by bit pattern: +-0, +-inf, +-max, normal and subnormal
    extremes, quiet and signalling NaNs of both signs with several payloads
    (each repeated many times, so stability is visible).  Specials are written
    through the integer view, so every NaN keeps its exact bits."""
    import numpy as np

    dt = np.dtype(dtype)
    ut = np.dtype(np.uint32 if dt.itemsize == 4 else np.uint64)
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal(n) * 100).astype(dt)
    if dt.itemsize == 4:
        nan_bits = [0x7FC00000, 0x7FC00001, 0x7FFFFFFF, 0x7F800001, 0x7FA00000,
                    0xFFC00000, 0xFFC00001, 0xFFFFFFFF, 0xFF800001]
    else:
        nan_bits = [0x7FF8000000000000, 0x7FF8000000000001, 0x7FFFFFFFFFFFFFFF, 0x7FF0000000000001,
                    0xFFF8000000000000, 0xFFF8000000000001, 0xFFFFFFFFFFFFFFFF, 0xFFF0000000000001]
    fi = np.finfo(dt)
    vals = np.array([0.0, -0.0, np.inf, -np.inf, fi.max, -fi.max, fi.tiny, -fi.tiny,
                     fi.tiny / 8, -fi.tiny / 8, fi.smallest_subnormal, -fi.smallest_subnormal], dtype=dt)
    specials = np.concatenate([np.array(nan_bits, dtype=ut), vals.view(ut)])
    idx = rng.integers(0, n, size=max(n // 4, 1))
    a.view(ut)[idx] = specials[rng.integers(0, specials.size, size=idx.size)]
    return a
