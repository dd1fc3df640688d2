"""DeviceSegmentReduce::Sum (CSR begin/end) on the GPU through the C ABI:
integers bit-exact against the oracle, floats within
|err_s| <= 1e-5 * sum_seg|x| of float64 sums, empty segments exactly +0.0."""
import numpy as np
import pytest

from conftest import golden, log
from oracle import oracle as o

pytestmark = pytest.mark.gpu

RTOL_SEG = 1e-5


def run(d_in, b, e, dtype):
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceSegmentReduce

    S = b.size
    out = g.empty(S, dtype)
    db, de = g.to_dev(b), g.to_dev(e)
    tmp = g.temp(DeviceSegmentReduce.GetTempStorageBytes(np.dtype(dtype).name, S))
    DeviceSegmentReduce().Sum(tmp, d_in, out, S, db, de)
    return g.to_host(out)


def test_kat_golden(gpu):
    # device_segment_reduce.cpp:62-125
    import gpu_util as g

    a = golden("segment_shuffled_1024_i32.bin", np.int32)
    b = golden("segment_shuffled_1024_begin_u32.bin", np.uint32)
    e = golden("segment_shuffled_1024_end_u32.bin", np.uint32)
    assert (run(g.to_dev(a), b, e, np.int32) == golden("segment_shuffled_1024_expect_i32.bin", np.int32)).all()


@pytest.mark.parametrize("dtype", [np.int32, np.uint32, np.int64, np.uint64])
@pytest.mark.parametrize("S", [1, 63, 64, 65, 257, 5000])
def test_integers_vs_oracle(gpu, dtype, S):
    import gpu_util as g

    n = 300_000
    b, e = o.segments(S, S + 1, n, S)
    a = g.random_array(dtype, n, seed=S)
    log(f"segment {np.dtype(dtype).name} S={S}")
    assert (run(g.to_dev(a), b, e, dtype) == o.segment_reduce(o.OP_SUM, a, b, e)).all()


def test_arbitrary_ranges_long_empty_inverted(gpu):
    import gpu_util as g

    rng = np.random.default_rng(9)
    n = 1 << 20
    S = 3000
    b = rng.integers(0, n, S).astype(np.uint32)
    L = rng.integers(0, 300, S)
    L[::50] = rng.integers(8193, 100_000, L[::50].size)  # long -> workgroup path
    L[::7] = 0
    e = np.minimum(b.astype(np.int64) + L, n).astype(np.uint32)
    e[::11] = b[::11] // 2  # inverted ranges -> empty
    a = g.random_array(np.int32, n, seed=1)
    assert (run(g.to_dev(a), b, e, np.int32) == o.segment_reduce(o.OP_SUM, a, b, e)).all()


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_floats_vs_float64(gpu, dtype):
    import gpu_util as g

    n = 1_000_000
    b, e = o.segments(5, 6, n, 7000)
    a = g.random_array(dtype, n, seed=4)
    got = run(g.to_dev(a), b, e, dtype)
    s, ab = o.segment_reduce_f64(a, b, e)
    assert (np.abs(got.astype(np.float64) - s) <= RTOL_SEG * ab + 1e-30).all()
    empty = b >= e
    assert empty.any() and all(np.asarray(x).tobytes() == np.zeros(1, dtype).tobytes() for x in got[empty])


def test_full_size_c5(gpu):
    # 2^27 float32 N(0,1), 2^20 CSR segments (geometric, mean 128, ~5 % empty)
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n, S = 1 << 27, 1 << 20
    log("segment f32 full 2^27 / 2^20")
    d = datagen.normal_f32(n, seed=datagen.SEED_SEG_VALUES)
    b, e = datagen.segments(n, S)
    ob, oe = o.segments(datagen.SEED_SEG_EMPTY, datagen.SEED_SEG_LEN, n, S)
    assert (b == ob).all() and (e == oe).all()
    got = run(d, b, e, np.float32)
    s, ab = o.segment_reduce_f64(g.to_host(d), b, e)
    assert (np.abs(got.astype(np.float64) - s) <= RTOL_SEG * ab).all()
    empty = b == e
    assert 0.03 < empty.mean() < 0.07
    assert (got[empty].view(np.uint32) == 0).all()  # +0.0 exactly
