"""DeviceScan::*ScanByKey / *SumByKey and DeviceReduce::ReduceByKey on the
GPU through the C ABI.  Integer values bit-exact against the oracle (itself
pinned against numpy cumsum differences / reduceat and the reference's
known answers); floating values within |err| <= 1e-5 * (sum of |x| over the
run prefix) of a float64 segmented scan / run sum."""
import numpy as np
import pytest

from conftest import golden, log
from oracle import oracle as o

pytestmark = pytest.mark.gpu

RTOL = 1e-5
KEY_DTYPES = [np.int32, np.uint32, np.float32, np.int64, np.uint64, np.float64]
VAL_DTYPES = [np.int32, np.uint32, np.float32, np.int64, np.uint64, np.float64]
OPS = {"sum": o.OP_SUM, "min": o.OP_MIN, "max": o.OP_MAX}
# tiles hold 8192 4-byte / 4096 8-byte values: cover both boundaries
SIZES = [1, 2, 63, 4095, 4096, 4097, 8191, 8192, 8193, 3 * 8192 + 5, 100_003]


def run_keys(n: int, mean_len: float, seed: int, dtype) -> np.ndarray:
    rng = np.random.default_rng(seed)
    heads = rng.random(n) < 1.0 / mean_len
    if n:
        heads[0] = True
    return (np.cumsum(heads) * 7 % 100_003).astype(dtype)


def values(dtype, n: int, seed: int) -> np.ndarray:
    dt = np.dtype(dtype)
    rng = np.random.default_rng(seed)
    if dt.kind == "f":
        return rng.standard_normal(n).astype(dt)
    info = np.iinfo(dt)
    return rng.integers(info.min, info.max, n, dtype=dt, endpoint=True)


def scan_by_key(kind, keys, vals, op="sum", init=0, pad=0, guard=0):
    """Runs the scan; returns (result, guard elements after the output)."""
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceScan

    n = vals.size
    s = DeviceScan()
    dk, dv = g.to_dev(keys, pad=pad), g.to_dev(vals, pad=pad)
    out = g.empty(n + guard, vals.dtype, pad=pad)
    if guard:
        out[n:].fill_(123)
    tmp = g.temp(DeviceScan.GetScanByKeyTempStorageBytes(keys.dtype.name, vals.dtype.name, n))
    if kind == "ExclusiveSumByKey" or kind == "InclusiveSumByKey":
        getattr(s, kind)(tmp, dk, dv, out, n)
    else:
        getattr(s, kind)(tmp, dk, dv, out, op, n, init)
    h = g.to_host(out)
    return h[:n], h[n:]


def reduce_by_key(keys, vals, op="sum", pad=0, guard=0):
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceReduce

    n = vals.size
    dk, dv = g.to_dev(keys, pad=pad), g.to_dev(vals, pad=pad)
    uk = g.empty(n + guard, keys.dtype, pad=pad)
    ag = g.empty(n + guard, vals.dtype, pad=pad)
    uk.fill_(0)
    ag.fill_(0)
    runs = g.empty(1, np.uint32)
    runs.fill_(0xDEAD)
    tmp = g.temp(DeviceReduce.GetReduceByKeyTempStorageBytes(keys.dtype.name, vals.dtype.name, n))
    DeviceReduce().ReduceByKey(tmp, dk, dv, uk, ag, runs, op, n)
    r = int(g.to_host(runs)[0])
    return g.to_host(uk), g.to_host(ag), r


def check_float_scan(got, keys, vals, inclusive):
    ref, ab = o.scan_by_key_f64(keys, vals, inclusive)
    err = np.abs(got.astype(np.float64) - ref)
    assert (err <= RTOL * ab + 1e-30).all(), float((err - RTOL * ab).max())


# ------------------------------------------------------------------ reference known answers
def test_kat_exclusive_sum_by_key_ones(gpu):
    # device_scan_test.cpp:111-167: keys i/100, values 1, N = 2^5..2^23 -> i % 100
    for i in range(5, 24):
        n = 1 << i
        log(f"scan_by_key KAT n={n}")
        keys = (np.arange(n) // 100).astype(np.int32)
        got, _ = scan_by_key("ExclusiveSumByKey", keys, np.ones(n, np.int32))
        assert (got == np.arange(n) % 100).all()


def test_kat_reduce_by_key_shuffled(gpu):
    # device_reduce_test.cpp:229-289: keys i/100 over the shuffled 0..4095
    a = golden("reduce_shuffled_4096_i32.bin", np.int32)
    keys = (np.arange(a.size) // 100).astype(np.int32)
    uk, ag, r = reduce_by_key(keys, a)
    assert r == 41
    assert (uk[:41] == np.arange(41)).all()
    assert (ag[:41] == np.array([a[i * 100:(i + 1) * 100].sum() for i in range(41)])).all()


# ------------------------------------------------------------------ parity sweeps
@pytest.mark.parametrize("kdt", KEY_DTYPES)
@pytest.mark.parametrize("vdt", VAL_DTYPES)
def test_scan_by_key_dtypes(gpu, kdt, vdt):
    n = 50_003
    for mean in (1.5, 300, 20_000):
        keys = run_keys(n, mean, 1, kdt)
        v = values(vdt, n, 2)
        for inclusive in (False, True):
            kind = "InclusiveSumByKey" if inclusive else "ExclusiveSumByKey"
            log(f"{kind} {np.dtype(kdt).name}/{np.dtype(vdt).name} mean={mean}")
            got, _ = scan_by_key(kind, keys, v)
            if np.dtype(vdt).kind == "f":
                check_float_scan(got, keys, v, inclusive)
            else:
                assert (got == o.scan_by_key(keys, v, inclusive)).all()


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("vdt", [np.int32, np.int64])
@pytest.mark.parametrize("pad", [0, 1])
def test_scan_by_key_sizes_and_alignment(gpu, n, vdt, pad):
    keys = run_keys(n, 40, n, np.int32)
    v = values(vdt, n, n + 1)
    for kind, inclusive in (("ExclusiveSumByKey", False), ("InclusiveSumByKey", True)):
        log(f"{kind} n={n} {np.dtype(vdt).name} pad={pad}")
        got, guard = scan_by_key(kind, keys, v, pad=pad, guard=64)
        assert (got == o.scan_by_key(keys, v, inclusive)).all()
        assert (guard == 123).all(), "write past the end of the output"


@pytest.mark.parametrize("op", ["sum", "min", "max"])
@pytest.mark.parametrize("vdt", [np.int32, np.uint32, np.float32, np.int64, np.float64])
def test_scan_by_key_ops_and_init(gpu, op, vdt):
    n = 70_001
    keys = run_keys(n, 50, 3, np.int64)
    dt = np.dtype(vdt)
    v = values(vdt, n, 4) if dt.kind != "f" else np.random.default_rng(4).integers(-1000, 1000, n).astype(dt)
    init = 7 if op != "max" else (-5 if dt.kind != "u" else 5)
    for inclusive in (False, True):
        kind = "InclusiveScanByKey" if inclusive else "ExclusiveScanByKey"
        log(f"{kind} op={op} {dt.name}")
        got, _ = scan_by_key(kind, keys, v, op, init)
        assert (got == o.scan_by_key(keys, v, inclusive, OPS[op], init)).all()


def test_scan_by_key_one_run_and_distinct_keys(gpu):
    # one run spanning ~120 tiles: every tile waits on the segmented (key,
    # value) look-back; decoupled_look_back.cpp:176-300 checks the same
    # combine over tiles that all share one key (exclusive prefix = the sum
    # of the tiles before)
    n = 1_000_003
    v = values(np.int32, n, 5)
    one = np.full(n, 3, np.uint32)
    for inclusive in (False, True):
        kind = "InclusiveSumByKey" if inclusive else "ExclusiveSumByKey"
        got, _ = scan_by_key(kind, one, v)
        assert (got == o.scan(v, inclusive)).all()
    distinct = np.arange(n, dtype=np.int64)
    got, _ = scan_by_key("ExclusiveScanByKey", distinct, v, "sum", 11)
    assert (got == 11).all()
    got, _ = scan_by_key("InclusiveScanByKey", distinct, v, "max", 0)
    assert (got == np.maximum(v, 0)).all()


def test_by_key_float_keys_zero_and_nan(gpu):
    keys = np.array([1.0, -0.0, 0.0, np.nan, np.nan, 2.0, 2.0], np.float32)
    v = np.ones(7, np.int32)
    got, _ = scan_by_key("InclusiveSumByKey", keys, v)
    assert list(got) == [1, 1, 2, 1, 1, 1, 2]
    uk, ag, r = reduce_by_key(keys, v)
    assert r == 5 and list(ag[:5]) == [1, 2, 1, 1, 2]


@pytest.mark.parametrize("kdt", KEY_DTYPES)
@pytest.mark.parametrize("vdt", VAL_DTYPES)
def test_reduce_by_key_dtypes(gpu, kdt, vdt):
    n = 60_007
    for mean in (1.5, 90, 30_000):
        keys = run_keys(n, mean, 6, kdt)
        v = values(vdt, n, 7)
        log(f"ReduceByKey {np.dtype(kdt).name}/{np.dtype(vdt).name} mean={mean}")
        uk, ag, r = reduce_by_key(keys, v)
        ek, ea = o.reduce_by_key(keys, v)
        assert r == ek.size
        assert uk[:r].tobytes() == ek.tobytes()
        if np.dtype(vdt).kind == "f":
            s, ab = o.reduce_by_key_f64(keys, v)
            assert (np.abs(ag[:r].astype(np.float64) - s) <= RTOL * ab + 1e-30).all()
        else:
            assert (ag[:r] == ea).all()


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("op", ["sum", "min", "max"])
def test_reduce_by_key_sizes_ops_guard(gpu, n, op):
    keys = run_keys(n, 6, n + 2, np.int32)
    v = values(np.int32, n, n + 3)
    log(f"ReduceByKey n={n} op={op}")
    uk, ag, r = reduce_by_key(keys, v, op, pad=1, guard=16)
    ek, ea = o.reduce_by_key(keys, v, OPS[op])
    assert r == ek.size
    assert (uk[:r] == ek).all() and (ag[:r] == ea).all()
    assert (uk[r:] == 0).all() and (ag[r:] == 0).all(), "write past the last run"


@pytest.mark.parametrize("vdt", [np.int32, np.float64])
@pytest.mark.parametrize("op", ["sum", "min", "max"])
def test_reduce_by_key_across_emit_groups(gpu, vdt, op):
    """Run counts and folds carried across the emit launch's groups of 64
    tiles: dense runs (every tile's staging area nearly full), runs longer
    than a group (whole groups without a head), and one run over everything."""
    tile = 8192 if np.dtype(vdt).itemsize == 4 else 4096
    n = 3 * 64 * tile + 4097
    for mean in (1.5, 1.5 * 64 * tile, float(n) * 10):
        keys = run_keys(n, mean, 8, np.int64)
        v = values(vdt, n, 9)
        log(f"ReduceByKey groups n={n} mean={mean:.0f} {np.dtype(vdt).name} {op}")
        uk, ag, r = reduce_by_key(keys, v, op, guard=8)
        ek, ea = o.reduce_by_key(keys, v, OPS[op])
        assert r == ek.size
        assert (uk[:r] == ek).all()
        if np.dtype(vdt).kind == "f" and op == "sum":
            s_, ab = o.reduce_by_key_f64(keys, v)
            assert (np.abs(ag[:r] - s_) <= RTOL * ab + 1e-30).all()
        else:
            assert (ag[:r] == ea).all()
        assert (uk[r:] == 0).all() and (ag[r:] == 0).all(), "write past the last run"


@pytest.mark.parametrize("op", ["sum", "max"])
def test_reduce_by_key_dense_and_sparse_tiles_mixed(gpu, op):
    """Tiles with more than 128 runs (processed again from the input with
    their prefixes) next to tiles that stage their runs: alternating regions
    of runs of mean 2 and mean 500, a single dense tile, and a tile with
    exactly 128 and 129 runs."""
    n = 40 * 8192 + 77
    rng = np.random.default_rng(11)
    mean = np.full(n, 500.0)
    mean[3 * 8192:9 * 8192] = 2.0        # dense tiles, crossing emit groups? (64-tile groups: no)
    mean[20 * 8192:21 * 8192] = 1.0      # one all-distinct tile
    mean[30 * 8192 + 100:31 * 8192] = 3.0
    heads = rng.random(n) < 1.0 / mean
    heads[0] = True
    # tile 12 with exactly 128 heads, tile 13 with 129
    for t, h in ((12, 128), (13, 129)):
        heads[t * 8192:(t + 1) * 8192] = False
        heads[t * 8192 + rng.choice(8192, h, replace=False)] = True
    keys = (np.cumsum(heads) * 3 % 65_521).astype(np.int32)
    v = values(np.int32, n, 12)
    log(f"ReduceByKey mixed dense/sparse tiles {op}")
    uk, ag, r = reduce_by_key(keys, v, op, guard=8)
    ek, ea = o.reduce_by_key(keys, v, OPS[op])
    assert r == ek.size
    assert (uk[:r] == ek).all() and (ag[:r] == ea).all()
    assert (uk[r:] == 0).all() and (ag[r:] == 0).all()


@pytest.mark.parametrize("kdt,vdt", [(np.int32, np.int32), (np.uint32, np.float32), (np.float32, np.int32),
                                     (np.int64, np.int64), (np.float64, np.float64), (np.uint64, np.float64),
                                     (np.int32, np.int64), (np.int64, np.int32)])
@pytest.mark.parametrize("op", ["sum", "min", "max"])
def test_reduce_by_key_direct_tile_densities(gpu, kdt, vdt, op):
    """Tiles with more than 128 runs write them out themselves.  When more
    than a quarter of a tile's elements start a run (and keys and values have
    one size) the runs go out through each wave slice's part of the tile's keys
    in LDS: slices with at most half as many runs as elements together at the
    end of the tile, denser ones at once.  Densities on both sides of both
    boundaries, every key distinct, a ragged last tile, the first tile (whose
    first head closes no run), and a guard past the outputs."""
    tile = 8192 if np.dtype(vdt).itemsize == 4 else 4096
    n = 5 * tile + 333
    for mean in (1.0, 1.6, 1.95, 2.0, 2.05, 2.5, 4.0, 16.0, 60.0):
        keys = np.arange(n).astype(kdt) if mean == 1.0 else run_keys(n, mean, int(mean * 100), kdt)
        v = values(vdt, n, 21)
        log(f"ReduceByKey direct tiles {np.dtype(kdt).name}/{np.dtype(vdt).name} mean={mean} {op}")
        uk, ag, r = reduce_by_key(keys, v, op, guard=8)
        ek, ea = o.reduce_by_key(keys, v, OPS[op])
        assert r == ek.size
        assert uk[:r].tobytes() == ek.tobytes()
        if np.dtype(vdt).kind == "f" and op == "sum":
            s_, ab = o.reduce_by_key_f64(keys, v)
            assert (np.abs(ag[:r].astype(np.float64) - s_) <= RTOL * ab + 1e-30).all()
        else:
            assert ag[:r].tobytes() == ea.tobytes()
        assert (uk[r:] == 0).all() and (ag[r:] == 0).all(), "write past the last run"


@pytest.mark.parametrize("n_staged_tiles", [15, 16, 17, 600, 3000, 5000])
def test_reduce_by_key_long_staged_prefix_then_dense(gpu, n_staged_tiles):
    """A long stretch of tiles that stage their runs (their batches of 8
    tiles never get an inclusive run count) followed by dense tiles, whose
    run-count walk adds up every batch of the stretch back to batch 0: the
    dense part starts at the last, first and second tile of a batch
    (15/16/17 tiles), and the walk takes one round trip of 64 batch words,
    two (600, 3000 tiles: the second one of 512 words) or three (5000)."""
    tile = 8192
    n = (n_staged_tiles + 6) * tile + 333
    rng = np.random.default_rng(n_staged_tiles)
    mean = np.full(n, 700.0)
    mean[n_staged_tiles * tile:] = 1.5  # dense from here on
    heads = rng.random(n) < 1.0 / mean
    heads[0] = True
    keys = np.cumsum(heads, dtype=np.int64).astype(np.uint32)
    v = values(np.uint32, n, 3)
    log(f"ReduceByKey {n_staged_tiles} staged tiles, then dense")
    uk, ag, r = reduce_by_key(keys, v, "sum", guard=8)
    ek, ea = o.reduce_by_key(keys, v)
    assert r == ek.size
    assert (uk[:r] == ek).all() and (ag[:r] == ea).all()
    assert (uk[r:] == 0).all() and (ag[r:] == 0).all()


def test_reduce_by_key_empty_and_single(gpu):
    uk, ag, r = reduce_by_key(np.empty(0, np.int32), np.empty(0, np.int32))
    assert r == 0
    uk, ag, r = reduce_by_key(np.array([9], np.int64), np.array([-4], np.int32))
    assert r == 1 and uk[0] == 9 and ag[0] == -4
    got, _ = scan_by_key("ExclusiveSumByKey", np.empty(0, np.int32), np.empty(0, np.int32))
    assert got.size == 0


# ------------------------------------------------------------------ full size (bench configuration)
def test_full_size_2p28(gpu):
    """ScanByKey / ReduceByKey over 2^28 int32 keys with geometric run lengths
    (mean 128) and int32 values, checked against the oracle."""
    import gpu_util as g
    import torch
    from lc_parallel_primitive_amd import DeviceReduce, DeviceScan

    n = 1 << 28
    w = o.gen("keys_u32", n, 0xB1)
    keys = np.cumsum((w & 127) == 0, dtype=np.int32)
    del w
    v = o.gen("reduce_i32", n, 0xB2)
    dk, dv = g.to_dev(keys), g.to_dev(v)
    out = torch.empty(n, dtype=torch.int32, device="cuda")
    tmp = g.temp(DeviceScan.GetScanByKeyTempStorageBytes("int32", "int32", n))
    log("InclusiveSumByKey int32 n=2^28")
    DeviceScan().InclusiveSumByKey(tmp, dk, dv, out, n)
    assert (g.to_host(out) == o.scan_by_key(keys, v, True)).all()
    del out, tmp
    uk = torch.empty(n, dtype=torch.int32, device="cuda")
    ag = torch.empty(n, dtype=torch.int32, device="cuda")
    runs = torch.zeros(1, dtype=torch.int32, device="cuda")
    tmp = g.temp(DeviceReduce.GetReduceByKeyTempStorageBytes("int32", "int32", n))
    log("ReduceByKey int32 n=2^28")
    DeviceReduce().ReduceByKey(tmp, dk, dv, uk, ag, runs, "sum", n)
    ek, ea = o.reduce_by_key(keys, v)
    r = int(g.to_host(runs)[0])
    assert r == ek.size
    assert (g.to_host(uk)[:r] == ek).all() and (g.to_host(ag)[:r] == ea).all()


def test_at_the_32_bit_limit(gpu):
    """n = 2^32 - 1 int32 keys in runs of 128 (key = index >> 7 of the 32-bit
    index; the last run holds 127) and int32 ones: ReduceByKey finds 2^25
    runs, each summing to its length, with the runs' keys; InclusiveSumByKey
    gives the position within the run plus one."""
    import torch

    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceReduce, DeviceScan, datagen

    n = (1 << 32) - 1
    log(f"ReduceByKey / InclusiveSumByKey int32 n={n}")
    dk = datagen.iota_u32(n).view(torch.int32)
    dk >>= 7
    dv = torch.ones(n, dtype=torch.int32, device="cuda")
    uk = torch.empty(n, dtype=torch.int32, device="cuda")
    ag = torch.empty(n, dtype=torch.int32, device="cuda")
    runs = torch.zeros(1, dtype=torch.int32, device="cuda")
    tmp = g.temp(DeviceReduce.GetReduceByKeyTempStorageBytes("int32", "int32", n))
    DeviceReduce().ReduceByKey(tmp, dk, dv, uk, ag, runs, "sum", n)
    r = int(runs.cpu()[0])
    assert r == 1 << 25
    assert bool((uk[:r] == dk[::128]).all())
    assert bool((ag[: r - 1] == 128).all()) and int(ag[r - 1]) == 127
    del uk, ag, tmp
    out = torch.empty(n, dtype=torch.int32, device="cuda")
    tmp = g.temp(DeviceScan.GetScanByKeyTempStorageBytes("int32", "int32", n))
    DeviceScan().InclusiveSumByKey(tmp, dk, dv, out, n)
    step = torch.arange(1, 129, dtype=torch.int32, device="cuda")
    full = n - 127
    assert bool((out[:full].view(-1, 128) == step).all())
    assert bool((out[full:] == step[:127]).all())
    del dk, dv, out, tmp
    torch.cuda.empty_cache()
