"""lcpp_scan_exclusive_sum_noalloc (the one entry point that allocates nothing:
its look-back state lives in a fixed device array inside the library) against
lcpp_scan_exclusive_sum on the same inputs, through the C ABI: integers
bit-exact, floats within the scans' normwise tolerance of a float64 host scan.
Two calls in a row share the array, the second on a smaller input; sizes past
the array's capacity are rejected before any launch."""
import ctypes

import numpy as np
import pytest

from conftest import log
from oracle import oracle as o

pytestmark = pytest.mark.gpu

SIZE_LIMIT = -6
MAX_N = {4: 65536 * 20480, 8: 32768 * 10240}  # tiles of the array x exclusive tile length


def _sp():
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("dtype", [np.uint32, np.int64, np.float32, np.float64])
def test_noalloc_matches_exclusive_sum_twice(gpu, dtype):
    import torch

    import gpu_util as g
    import lc_parallel_primitive_amd as lcpp

    L = lcpp.lib()
    code = lcpp._capi.dtype_code(np.dtype(dtype).name)
    for n in (3_000_017, 100_003):  # the second call is smaller: nothing may leak from the first
        a = g.random_array(dtype, n, seed=n)
        if np.dtype(dtype).kind == "f":
            a = (np.random.default_rng(n).standard_normal(n)).astype(dtype)
        d = g.to_dev(a)
        guard = 4096
        out = g.empty(n + guard, dtype)
        out.view(torch.uint8).fill_(7)
        log(f"noalloc scan {np.dtype(dtype).name} n={n}")
        assert L.lcpp_scan_exclusive_sum_noalloc(code, _p(d), _p(out), n, _sp()) == 0
        b = ctypes.c_size_t()
        assert L.lcpp_scan_temp_bytes(code, n, ctypes.byref(b)) == 0
        t = g.temp(b.value)
        ref = g.empty(n, dtype)
        assert L.lcpp_scan_exclusive_sum(code, _p(t), b.value, _p(d), _p(ref), n, _sp()) == 0
        got, want = g.to_host(out), g.to_host(ref)
        assert (got[n:].view(np.uint8) == 7).all()  # nothing written past n
        got = got[:n]
        if np.dtype(dtype).kind in "iu":
            assert got.tobytes() == want.tobytes()
            assert got.tobytes() == o.scan(a, inclusive=False).tobytes()
        else:
            exact, absp = o.scan_f64(a, inclusive=False)
            tol = 1e-5 * absp + 1e-30
            assert (np.abs(got.astype(np.float64) - exact) <= tol).all()
            assert (np.abs(want.astype(np.float64) - exact) <= tol).all()


def test_noalloc_at_capacity_and_past_it(gpu):
    import torch

    import gpu_util as g
    import lc_parallel_primitive_amd as lcpp

    L = lcpp.lib()
    n = MAX_N[8]  # int64 at exactly the array's capacity
    log(f"noalloc scan int64 n={n} (capacity)")
    d = torch.randint(-1000, 1000, (n,), dtype=torch.int64, device="cuda")
    out = torch.empty_like(d)
    assert L.lcpp_scan_exclusive_sum_noalloc(3, _p(d), _p(out), n, _sp()) == 0
    want = torch.cumsum(d, 0) - d
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    del want
    # one more tile than the array holds: rejected before any launch
    assert L.lcpp_scan_exclusive_sum_noalloc(3, _p(d), _p(out), n + 10240, _sp()) == SIZE_LIMIT
    assert L.lcpp_scan_exclusive_sum_noalloc(1, _p(d), _p(out), MAX_N[4] + 1, _sp()) == SIZE_LIMIT
    assert L.lcpp_scan_exclusive_sum_noalloc(1, None, _p(out), 10, _sp()) == -1
    assert L.lcpp_scan_exclusive_sum_noalloc(9, _p(d), _p(out), 10, _sp()) == -3
    assert L.lcpp_scan_exclusive_sum_noalloc(1, None, None, 0, _sp()) == 0
    # and a regular-size call afterwards is exact again
    small = g.random_array(np.uint32, 50_000, seed=9)
    ds, os_ = g.to_dev(small), g.empty(50_000, np.uint32)
    assert L.lcpp_scan_exclusive_sum_noalloc(1, _p(ds), _p(os_), 50_000, _sp()) == 0
    assert g.to_host(os_).tobytes() == o.scan(small, inclusive=False).tobytes()
