"""DeviceScan::ExclusiveSum/InclusiveSum and ExclusiveScan/InclusiveScan
(Sum/Min/Max with an initial value) on the GPU through the C ABI: integers
bit-exact (wraparound) against the oracle, floats within
|y_i - yhat_i| <= 1e-5 * sum_{j<=i}|x_j| of a float64 scan."""
import numpy as np
import pytest

from conftest import log
from oracle import oracle as o

pytestmark = pytest.mark.gpu

RTOL_SCAN = 1e-5
INT_DTYPES = [np.int32, np.uint32, np.int64, np.uint64]


def run(kind, d_in, n, dtype, tmp=None, pad=0):
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceScan

    s = DeviceScan()
    out = g.empty(n, dtype, pad=pad)
    if tmp is None:
        tmp = g.temp(DeviceScan.GetTempStorageBytes(np.dtype(dtype).name, n))
    getattr(s, kind)(tmp, d_in, out, n)
    return g.to_host(out)


def test_kat_ones_reused_temp(gpu):
    # device_scan_test.cpp:67-108: ones, N = 2^0..2^23, one temp buffer for both scans
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceScan

    for i in range(24):
        n = 1 << i
        log(f"scan ones n={n}")
        d = g.to_dev(np.ones(n, np.uint32))
        tmp = g.temp(DeviceScan.GetTempStorageBytes("uint32", n))
        assert (run("ExclusiveSum", d, n, np.uint32, tmp) == np.arange(n, dtype=np.uint32)).all()
        assert (run("InclusiveSum", d, n, np.uint32, tmp) == np.arange(1, n + 1, dtype=np.uint32)).all()


@pytest.mark.parametrize("dtype", INT_DTYPES)
# exclusive tiles hold 20480 32-bit / 10240 64-bit elements, inclusive ones 16384 /
# 8192 (24576 for float): cover every boundary
@pytest.mark.parametrize("n", [1, 2, 4097, 8191, 8192, 8193, 10239, 10240, 10241, 16383, 16384, 16385,
                               20479, 20480, 20481, 24575, 24576, 24577, 3 * 16384 + 5,
                               3 * 20480 + 5, 3 * 24576 + 5, 100_003, 1 << 20])
@pytest.mark.parametrize("pad", [0, 1])
def test_integers_vs_oracle(gpu, dtype, n, pad):
    import gpu_util as g

    a = g.random_array(dtype, n, seed=n + pad)
    log(f"scan {np.dtype(dtype).name} n={n} pad={pad}")
    d = g.to_dev(a, pad=pad)
    assert (run("ExclusiveSum", d, n, dtype, pad=pad) == o.scan(a, False)).all()
    assert (run("InclusiveSum", d, n, dtype, pad=pad) == o.scan(a, True)).all()


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("n", [1, 4097, 24577, 3 * 24576 + 5, 1_000_003])
def test_floats_vs_float64(gpu, dtype, n):
    import gpu_util as g

    a = g.random_array(dtype, n, seed=7)
    d = g.to_dev(a)
    for kind, incl in (("ExclusiveSum", False), ("InclusiveSum", True)):
        got = run(kind, d, n, dtype).astype(np.float64)
        ref, ab = o.scan_f64(a, incl)
        assert (np.abs(got - ref) <= RTOL_SCAN * ab + 1e-30).all()


def test_full_size_u32_exclusive_wraparound(gpu):
    # BASELINE config C2a: 2^28 uint32 in [0, 255]; the total (~3.4e10) wraps mod 2^32
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 1 << 28
    log("scan u32 exclusive full 2^28")
    d = datagen.u8_u32(n)
    got = run("ExclusiveSum", d, n, np.uint32)
    h = g.to_host(d)
    inc = np.cumsum(h, dtype=np.uint32)
    assert got[0] == 0 and (got[1:] == inc[:-1]).all()
    assert int(inc[-1]) == int(h.astype(np.uint64).sum()) % (1 << 32)


def test_full_size_f32_inclusive(gpu):
    # BASELINE config C2b: 2^28 float32 N(0,1), against a float64 scan
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 1 << 28
    log("scan f32 inclusive full 2^28")
    d = datagen.normal_f32(n)
    got = run("InclusiveSum", d, n, np.float32)
    h = g.to_host(d).astype(np.float64)
    ref = np.cumsum(h)
    ab = np.cumsum(np.abs(h))
    err = np.abs(got.astype(np.float64) - ref)
    assert (err <= RTOL_SCAN * ab).all(), float((err / ab).max())


@pytest.mark.parametrize("dtype", [np.uint32, np.int64])
@pytest.mark.parametrize("n", [5, 10241, 16383, 16385, 20479, 24577, 3 * 16384 + 7])
@pytest.mark.parametrize("pad", [0, 1])
def test_ragged_tile_writes_nothing_past_the_end(gpu, dtype, n, pad):
    """The last tile's element-wise path stores only [0, n): the output's
    trailing guard (and the input's, so every access stays inside allocated
    memory even past n) keeps its fill value."""
    import gpu_util as g
    import torch

    guard = 1 << 15  # > one tile of elements
    a = g.random_array(dtype, n, seed=n)
    din = g.empty(n + guard, dtype, pad=pad)
    din[:n].copy_(torch.from_numpy(a))
    din[n:].fill_(1)
    for kind, incl in (("ExclusiveSum", False), ("InclusiveSum", True)):
        log(f"scan guard {kind} {np.dtype(dtype).name} n={n} pad={pad}")
        out = g.empty(n + guard, dtype, pad=pad)
        out.fill_(77)
        from lc_parallel_primitive_amd import DeviceScan

        tmp = g.temp(DeviceScan.GetTempStorageBytes(np.dtype(dtype).name, n))
        getattr(DeviceScan(), kind)(tmp, din, out, n)
        h = g.to_host(out)
        assert (h[:n] == o.scan(a, incl)).all()
        assert (h[n:] == 77).all(), "store past the end of the output"


@pytest.mark.parametrize("kind", ["ExclusiveSum", "InclusiveSum"])
def test_past_2p32_elements_ones(gpu, kind):
    """n = 2^32 + 12345 uint32 ones (16 GiB; element offsets and positions
    past 32 bits): the scan of ones is the index (exclusive) or the index
    plus one (inclusive) mod 2^32, compared on the device against the
    generator's 32-bit index."""
    import torch

    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceScan, datagen

    n = (1 << 32) + 12345
    log(f"scan u32 {kind} ones n={n}")
    d = torch.ones(n, dtype=torch.int32, device="cuda").view(torch.uint32)
    out = torch.empty(n, dtype=torch.uint32, device="cuda")
    tmp = g.temp(DeviceScan.GetTempStorageBytes("uint32", n))
    getattr(DeviceScan(), kind)(tmp, d, out, n)
    del d, tmp
    idx = datagen.iota_u32(n)
    o = out.view(torch.int32)
    if kind == "ExclusiveSum":
        ok = bool((o == idx.view(torch.int32)).all())
    else:
        ok = bool((o[:-1] == idx.view(torch.int32)[1:]).all()) and int(o[-1]) == (n & 0xFFFFFFFF)
    del out, idx, o
    torch.cuda.empty_cache()
    assert ok


# ------------------------------------------------------------------ ExclusiveScan / InclusiveScan (op, init)
ALL_DTYPES = [np.int32, np.uint32, np.float32, np.int64, np.uint64, np.float64]
SCAN_OPS = {"sum": o.OP_SUM, "min": o.OP_MIN, "max": o.OP_MAX}


def run_op(kind, d_in, n, dtype, op, init, pad=0):
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceScan

    out = g.empty(n, dtype, pad=pad)
    tmp = g.temp(DeviceScan.GetTempStorageBytes(np.dtype(dtype).name, n))
    getattr(DeviceScan(), kind)(tmp, d_in, out, n, op, init)
    return g.to_host(out)


def op_init(dtype, op):
    """An initial value that changes the results: inside the data's range for
    Min/Max, far from zero for Sum."""
    if np.dtype(dtype).kind == "f":
        return {"sum": 1.0e4, "min": -20.0, "max": 20.0}[op]
    info = np.iinfo(dtype)
    return {"sum": int(info.max // 7), "min": int(info.min // 2 + info.max // 2), "max": int(info.max // 3)}[op]


@pytest.mark.parametrize("dtype", ALL_DTYPES)
@pytest.mark.parametrize("op", ["sum", "min", "max"])
@pytest.mark.parametrize("n", [1, 8191, 8193, 16385, 20481, 24577, 3 * 20480 + 5, 100_003])
@pytest.mark.parametrize("pad", [0, 1])
def test_scan_op_init_vs_oracle(gpu, dtype, op, n, pad):
    """Integers (and float Min/Max: no rounding) bit-exact against the
    oracle; float sums within 1e-5 * (|init| + sum_{j<=i}|x_j|) of a float64
    scan.  Ragged last tiles, misaligned pointers (pad = 1)."""
    import gpu_util as g

    a = g.random_array(dtype, n, seed=n + pad + len(op))
    init = op_init(dtype, op)
    log(f"scan op={op} init={init} {np.dtype(dtype).name} n={n} pad={pad}")
    d = g.to_dev(a, pad=pad)
    for kind, incl in (("ExclusiveScan", False), ("InclusiveScan", True)):
        got = run_op(kind, d, n, dtype, op, init, pad=pad)
        if np.dtype(dtype).kind == "f" and op == "sum":
            ref, ab = o.scan_f64(a, incl)
            err = np.abs(got.astype(np.float64) - (ref + init))
            assert (err <= RTOL_SCAN * (ab + abs(init)) + 1e-30).all(), kind
        elif np.dtype(dtype).kind == "f":
            # Min/Max of -0.0 and +0.0 return either zero depending on the fold order
            assert np.array_equal(got, o.scan_op(a, incl, SCAN_OPS[op], init)), kind
        else:
            assert got.tobytes() == o.scan_op(a, incl, SCAN_OPS[op], init).tobytes(), kind


@pytest.mark.parametrize("kind", ["ExclusiveScan", "InclusiveScan"])
def test_scan_op_identity_init_equals_sum_scan(gpu, kind):
    """Sum with init 0 is ExclusiveSum / InclusiveSum, bit for bit (integers)."""
    import gpu_util as g

    n = 200_001
    a = g.random_array(np.int64, n, seed=3)
    d = g.to_dev(a)
    got = run_op(kind, d, n, np.int64, "sum", 0)
    assert (got == run(kind.replace("Scan", "Sum"), d, n, np.int64)).all()


@pytest.mark.parametrize("op", ["min", "max"])
def test_scan_op_full_size_u32(gpu, op):
    """2^28 uint32 running Min / Max from an init inside the data's range,
    against numpy's minimum / maximum.accumulate (with init prepended)."""
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 1 << 28
    log(f"scan u32 inclusive {op} full 2^28")
    d = datagen.keys_u32(n)
    init = 0x7FFFFFFF
    got = run_op("InclusiveScan", d, n, np.uint32, op, init)
    h = g.to_host(d)
    npop = np.minimum if op == "min" else np.maximum
    ref = npop.accumulate(np.concatenate([np.array([init], np.uint32), h]), dtype=np.uint32)[1:]
    assert (got == ref).all()


def test_scan_op_sum_full_size_exclusive_with_init(gpu):
    """2^28 uint32 in [0, 255] with init 2^32 - 5: wraps at once, bit-exact."""
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 1 << 28
    log("scan u32 exclusive sum init full 2^28")
    d = datagen.u8_u32(n)
    init = (1 << 32) - 5
    got = run_op("ExclusiveScan", d, n, np.uint32, "sum", init)
    h = g.to_host(d)
    inc = np.cumsum(h, dtype=np.uint32) + np.uint32(init)
    assert got[0] == init and (got[1:] == inc[:-1]).all()
