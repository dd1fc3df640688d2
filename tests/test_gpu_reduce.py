"""DeviceReduce::Sum/Min/Max/ArgMin/ArgMax/TransformReduce on the GPU through
the C ABI, against the oracle
(bit-exact for integers; float sums within |err| <= 1e-5 * sum|x| of a
float64 reduction)."""
import numpy as np
import pytest

from conftest import golden, log
from oracle import oracle as o

pytestmark = pytest.mark.gpu

RTOL_SUM = 1e-5  # normwise: |err| <= RTOL_SUM * sum(|x|)
DTYPES = [np.int32, np.uint32, np.float32, np.int64, np.uint64, np.float64]


def run(op, a_dev, n, dtype):
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceReduce

    r = DeviceReduce()
    out = g.empty(1, dtype)
    tmp = g.temp(DeviceReduce.GetTempStorageBytes(np.dtype(dtype).name, n))
    getattr(r, op)(tmp, a_dev, out, n)
    return g.to_host(out)[0]


def test_kat_sum_of_ones(gpu):
    # device_reduce_test.cpp:66-90: Sum<uint> of N ones == N, N = 2^k + 1, k < 24
    import gpu_util as g

    for k in range(24):
        n = (1 << k) + 1
        log(f"reduce ones n={n}")
        assert run("Sum", g.to_dev(np.ones(n, np.uint32)), n, np.uint32) == n


def test_kat_min_max_shuffled(gpu):
    # device_reduce_test.cpp:120-166
    import gpu_util as g

    a = golden("reduce_shuffled_4096_i32.bin", np.int32)
    exp = golden("reduce_shuffled_4096_expect_min_max_sum_i32.bin", np.int32)
    d = g.to_dev(a)
    assert run("Min", d, a.size, np.int32) == exp[0]
    assert run("Max", d, a.size, np.int32) == exp[1]
    assert run("Sum", d, a.size, np.int32) == exp[2]


# tiles hold 32768 4-byte / 16384 8-byte elements (12288 / 6144 for Arg*); at
# 20M elements the grid is at its 512-workgroup cap with a ragged last chunk
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1, 63, 4097, 16384, 16385, 32768, 32769, 1_000_003, 20_000_003])
@pytest.mark.parametrize("pad", [0, 1])
def test_all_dtypes_vs_oracle(gpu, dtype, n, pad):
    import gpu_util as g

    a = g.random_array(dtype, n, seed=n)
    log(f"reduce {np.dtype(dtype).name} n={n} pad={pad}")
    d = g.to_dev(a, pad=pad)
    for op, code in (("Min", o.OP_MIN), ("Max", o.OP_MAX)):
        assert run(op, d, n, dtype) == o.reduce(code, a)
    got = run("Sum", d, n, dtype)
    if np.dtype(dtype).kind == "f":
        s, ab = o.reduce_f64(a)
        assert abs(float(got) - s) <= RTOL_SUM * ab + 1e-30
    else:
        assert got == o.reduce(o.OP_SUM, a)


def test_empty_gives_init(gpu):
    import gpu_util as g

    d = g.empty(4, np.int32)
    assert run("Sum", d, 0, np.int32) == 0
    assert run("Min", d, 0, np.int32) == np.iinfo(np.int32).max
    f = g.empty(4, np.float32)
    assert run("Max", f, 0, np.float32) == np.finfo(np.float32).min  # lowest(), not min()


def test_float_max_all_negative(gpu):
    # The reference's Max init numeric_limits<float>::min() would return 1.17e-38 here.
    import gpu_util as g

    a = -np.abs(g.random_array(np.float32, 10_000, 5)) - 1
    assert run("Max", g.to_dev(a), a.size, np.float32) == a.max()


def test_float_sum_deterministic(gpu):
    from lc_parallel_primitive_amd import datagen

    n = 1 << 24
    d = datagen.normal_f32(n)
    r1, r2 = run("Sum", d, n, np.float32), run("Sum", d, n, np.float32)
    assert np.float32(r1).tobytes() == np.float32(r2).tobytes()


@pytest.mark.parametrize("lg", [24, 28])
def test_full_size_int32_closed_form(gpu, lg):
    # BASELINE config C1 (2^24) and the north-star size (2^28): uniform [-1000, 1000]
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 1 << lg
    log(f"reduce int32 full n=2^{lg}")
    d = datagen.reduce_i32(n)
    got = run("Sum", d, n, np.int32)
    h = g.to_host(d)
    exact = int(h.astype(np.int64).sum())
    assert int(got) == (exact + (1 << 31)) % (1 << 32) - (1 << 31)
    assert run("Min", d, n, np.int32) == -1000 and run("Max", d, n, np.int32) == 1000
    # spot-check the generator against the oracle's host restatement
    assert (h[:4096] == o.gen("reduce_i32", 4096, datagen.SEED_REDUCE)).all()


def test_full_size_float32(gpu):
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 1 << 28
    d = datagen.normal_f32(n)
    got = run("Sum", d, n, np.float32)
    s, ab = o.reduce_f64(g.to_host(d))
    assert abs(float(got) - s) <= RTOL_SUM * ab


# ------------------------------------------------------------------ ArgMin / ArgMax
def run_arg(is_max, d_in, n, dtype):
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceReduce

    out = g.empty(1, dtype)
    idx = g.empty(1, np.uint32)
    tmp = g.temp(DeviceReduce.GetArgTempStorageBytes(np.dtype(dtype).name, n))
    (DeviceReduce().ArgMax if is_max else DeviceReduce().ArgMin)(tmp, d_in, out, idx, n)
    return g.to_host(out)[0], int(g.to_host(idx)[0])


def test_arg_kat_shuffled(gpu):
    # device_reduce_test.cpp:169-225: shuffled 0..4095, std::min_element / max_element
    import gpu_util as g

    a = golden("reduce_shuffled_4096_i32.bin", np.int32)
    d = g.to_dev(a)
    assert run_arg(False, d, a.size, np.int32) == (0, int(np.nonzero(a == 0)[0][0]))
    assert run_arg(True, d, a.size, np.int32) == (4095, int(np.nonzero(a == 4095)[0][0]))


# Arg* tiles hold 12288 4-byte / 6144 8-byte elements; at 20M elements the
# grid is at its 1024-workgroup cap with a ragged last chunk
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1, 63, 4097, 6144, 6145, 12288, 12289, 32768, 1_000_003, 20_000_003])
def test_arg_vs_oracle_with_ties(gpu, dtype, n):
    import gpu_util as g

    rng = np.random.default_rng(n)
    a = rng.integers(0, 97, size=n).astype(dtype)  # many ties: the index rule decides
    log(f"argmin/argmax {np.dtype(dtype).name} n={n}")
    d = g.to_dev(a)
    for is_max in (False, True):
        v, i = run_arg(is_max, d, n, dtype)
        ev, ei = o.reduce_arg(is_max, a)
        assert (v, i) == (ev, ei)


def test_arg_empty(gpu):
    import gpu_util as g

    d = g.empty(4, np.int32)
    assert run_arg(False, d, 0, np.int32) == (np.iinfo(np.int32).max, 0xFFFFFFFF)
    f = g.empty(4, np.float32)
    assert run_arg(True, f, 0, np.float32) == (np.finfo(np.float32).min, 0)


def test_arg_full_size_int32(gpu):
    # 2^28 values in [-1000, 1000]: ArgMin = first -1000, ArgMax = last 1000
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 1 << 28
    log("argmin/argmax int32 full 2^28")
    d = datagen.reduce_i32(n)
    h = g.to_host(d)
    assert run_arg(False, d, n, np.int32) == (-1000, int(np.argmin(h)))
    assert run_arg(True, d, n, np.int32) == (1000, n - 1 - int(np.argmax(h[::-1])))


# ------------------------------------------------------------------ TransformReduce
def run_transform(op, xf, d_in, n, dtype, init):
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceReduce

    out = g.empty(1, dtype)
    tmp = g.temp(DeviceReduce.GetTempStorageBytes(np.dtype(dtype).name, n))
    DeviceReduce().TransformReduce(tmp, d_in, out, n, op, xf, init)
    return g.to_host(out)[0]


OPS = {"sum": o.OP_SUM, "min": o.OP_MIN, "max": o.OP_MAX}
XFS = {"identity": o.XF_IDENTITY, "negate": o.XF_NEGATE, "abs": o.XF_ABS, "square": o.XF_SQUARE}


def test_transform_kat_max_of_squares(gpu):
    # device_reduce_test.cpp:92-117
    import gpu_util as g

    a = golden("reduce_shuffled_4096_i32.bin", np.int32)
    assert run_transform("max", "square", g.to_dev(a), a.size, np.int32, 0) == 4095 * 4095


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("op", list(OPS))
@pytest.mark.parametrize("xf", list(XFS))
def test_transform_vs_oracle(gpu, dtype, op, xf):
    import gpu_util as g

    n = 300_007
    a = g.random_array(dtype, n, seed=17)
    d = g.to_dev(a)
    init = np.array([3], dtype=dtype)[0]
    got = run_transform(op, xf, d, n, dtype, init)
    if np.dtype(dtype).kind == "f" and op == "sum":
        t = {"identity": a, "negate": -a, "abs": np.abs(a), "square": a * a}[xf].astype(np.float64)
        s, ab = float(t.sum()) + float(init), float(np.abs(t).sum()) + abs(float(init))
        assert abs(float(got) - s) <= RTOL_SUM * ab
    else:
        assert got == o.reduce_transform(OPS[op], XFS[xf], a, init)


@pytest.mark.parametrize("dtype", [np.int32, np.uint64, np.float64])
@pytest.mark.parametrize("op", list(OPS))
def test_reduce_with_initial_value(gpu, dtype, op):
    """DeviceReduce::Reduce(reduce_op, initial_value) (device_reduce.h:131-147):
    the oracle's fold from init (integers exact), floats against float64."""
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceReduce

    n = 100_003
    a = g.random_array(dtype, n, seed=23)
    d = g.to_dev(a)
    out = g.empty(1, dtype)
    init = np.array([-5 if np.dtype(dtype).kind != "u" else 5], dtype=dtype)[0]
    tmp = g.temp(DeviceReduce.GetTempStorageBytes(np.dtype(dtype).name, n))
    DeviceReduce().Reduce(tmp, d, out, n, op, init)
    got = g.to_host(out)[0]
    if np.dtype(dtype).kind == "f" and op == "sum":
        t = a.astype(np.float64)
        s, ab = float(t.sum()) + float(init), float(np.abs(t).sum()) + abs(float(init))
        assert abs(float(got) - s) <= RTOL_SUM * ab
    else:
        assert got == o.reduce_transform(OPS[op], o.XF_IDENTITY, a, init)


def test_past_2p32_elements(gpu):
    """Sum of n = 2^32 + 12345 int32 ones wraps to 12345; ArgMax/ArgMin over
    n = 2^32 - 1 elements (the most that 32-bit indices allow): ties of ones
    go to the last / first index, and a lone 0 at the last index is found."""
    import torch

    n = (1 << 32) + 12345
    log(f"reduce int32 ones n={n}")
    d = torch.ones(n, dtype=torch.int32, device="cuda")
    assert int(run("Sum", d, n, np.int32)) == 12345
    m = (1 << 32) - 1
    assert run_arg(True, d, m, np.int32) == (1, m - 1)
    assert run_arg(False, d, m, np.int32) == (1, 0)
    d[m - 1] = 0
    assert run_arg(False, d, m, np.int32) == (0, m - 1)
    del d
    torch.cuda.empty_cache()
