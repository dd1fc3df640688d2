"""Seeded randomized parity cases for every primitive: random sizes (1 to
2^20, log-uniform, plus 4 cases per group between 2^22 and 2^26), integer dtypes, value distributions (uniform, few
distinct, AND-of-3, constant), sort directions, run lengths (one to three
per input, for by-key) and segment
layouts (tiling, random order, random windows with overlaps, gaps and
inverted ranges).  Integer data, so every result is exact against the
oracle.  A larger sweep of this kind (sizes to 2^25) found the gather load
whose offset wrapped below zero (see test_gather_lowest_segment_late_in_wave)."""
import numpy as np
import pytest

from conftest import log
from oracle import oracle as o

pytestmark = pytest.mark.gpu

INT_DTYPES = [np.int32, np.uint32, np.int64, np.uint64]
# Sizes are log-uniform in [2^LOG2_RANGE[0], 2^LOG2_RANGE[1]); every group
# also runs LARGE_CASES seeds in LOG2_LARGE (the regime where a wrapped gather
# offset once showed: ~3e7 elements).
LOG2_RANGE = (0, 20)
LOG2_LARGE = (22, 26)
LARGE_CASES = 4


def cases(n_small):
    """(seed, log2 size range) pairs: n_small small cases, then the large ones."""
    return [(s, LOG2_RANGE) for s in range(n_small)] + [(100 + s, LOG2_LARGE) for s in range(LARGE_CASES)]


def values(rng, dt, n, kind):
    info = np.iinfo(dt)

    def uni():
        return rng.integers(info.min, info.max, size=n, dtype=dt, endpoint=True)

    if kind == 0:
        return uni()
    if kind == 1:
        return rng.integers(0, 7, size=n).astype(dt)
    if kind == 2:
        return uni() & uni() & uni()
    return np.full(n, rng.integers(info.min, info.max, dtype=dt, endpoint=True), dtype=dt)


def case_params(seed, log2_range=LOG2_RANGE):
    rng = np.random.default_rng(seed)
    n = int(np.exp(rng.uniform(log2_range[0] * np.log(2), log2_range[1] * np.log(2))))
    return rng, n, INT_DTYPES[rng.integers(0, 4)], int(rng.integers(0, 4))


@pytest.mark.parametrize("seed,lr", cases(24))
def test_random_reduce_and_scan(gpu, seed, lr):
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceReduce, DeviceScan

    rng, n, dt, kind = case_params(1000 + seed, lr)
    a = values(rng, dt, n, kind)
    log(f"random reduce/scan seed={seed} n={n} {np.dtype(dt).name} kind={kind}")
    d = g.to_dev(a)
    out = g.empty(1, dt)
    r = DeviceReduce()
    tmp = g.temp(DeviceReduce.GetTempStorageBytes(np.dtype(dt).name, n))
    for nm, op in (("Sum", o.OP_SUM), ("Min", o.OP_MIN), ("Max", o.OP_MAX)):
        getattr(r, nm)(tmp, d, out, n)
        assert g.to_host(out)[0] == o.reduce(op, a), nm
    idx = g.empty(1, np.uint32)
    tmpa = g.temp(DeviceReduce.GetArgTempStorageBytes(np.dtype(dt).name, n))
    for nm, is_max in (("ArgMin", False), ("ArgMax", True)):
        getattr(r, nm)(tmpa, d, out, idx, n)
        v, i = o.reduce_arg(is_max, a)
        assert g.to_host(out)[0] == v and g.to_host(idx)[0] == i, nm
    so = g.empty(n, dt)
    s = DeviceScan()
    tmps = g.temp(DeviceScan.GetTempStorageBytes(np.dtype(dt).name, n))
    for inclusive in (False, True):
        (s.InclusiveSum if inclusive else s.ExclusiveSum)(tmps, d, so, n)
        assert (g.to_host(so) == o.scan(a, inclusive)).all(), inclusive
    op = ["sum", "min", "max"][seed % 3]
    init = values(rng, dt, 1, 0)[0]
    for inclusive in (False, True):
        (s.InclusiveScan if inclusive else s.ExclusiveScan)(tmps, d, so, n, op, init)
        ref = o.scan_op(a, inclusive, {"sum": o.OP_SUM, "min": o.OP_MIN, "max": o.OP_MAX}[op], init)
        assert (g.to_host(so) == ref).all(), (op, inclusive)


@pytest.mark.parametrize("seed,lr", cases(24))
def test_random_sorts(gpu, seed, lr):
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceRadixSort

    rng, n, dt, kind = case_params(2000 + seed, lr)
    a = values(rng, dt, n, kind)
    desc = bool(rng.integers(0, 2))
    vdt = [np.uint32, np.uint64][rng.integers(0, 2)]
    v = np.arange(n, dtype=vdt)
    log(f"random sort seed={seed} n={n} {np.dtype(dt).name} kind={kind} desc={desc}")
    s = DeviceRadixSort()
    ko = g.empty(n, dt)
    tmp = g.temp(DeviceRadixSort.GetSortKeysTempStorageBytes(np.dtype(dt).name, n))
    (s.SortKeysDescending if desc else s.SortKeys)(tmp, g.to_dev(a), ko, n)
    assert (g.to_host(ko) == o.radix_sort(a, descending=desc)).all()
    vo = g.empty(n, vdt)
    tmp = g.temp(DeviceRadixSort.GetSortPairsTempStorageBytes(np.dtype(dt).name, np.dtype(vdt).name, n))
    (s.SortPairsDescending if desc else s.SortPairs)(tmp, g.to_dev(a), ko, g.to_dev(v), vo, n)
    rk, rv = o.radix_sort(a, v, descending=desc)
    assert (g.to_host(ko) == rk).all() and (g.to_host(vo) == rv).all()


@pytest.mark.parametrize("seed,lr", cases(24))
def test_random_by_key(gpu, seed, lr):
    import torch

    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceReduce, DeviceScan

    rng, n, dt, kind = case_params(3000 + seed, lr)
    vdt = [np.int32, np.int64][int(rng.integers(0, 2))]
    # run lengths: one per piece of the input, 1 to 3 pieces (so stretches of
    # tiles that stage their runs meet stretches of tiles that write them)
    pieces = int(rng.integers(1, 4))
    bnd = np.concatenate([[0], np.sort(rng.integers(0, n + 1, size=pieces - 1)), [n]])
    runs = [int(rng.integers(1, 8)) if rng.random() < 0.5 else int(rng.integers(1, 400)) for _ in range(pieces)]
    keys = np.concatenate([np.repeat(rng.integers(0, 4, size=(b - a) // r + 1), r)[:b - a]
                           for a, b, r in zip(bnd[:-1], bnd[1:], runs)]).astype(dt)
    vals = values(rng, vdt, n, 1)
    op = ["sum", "min", "max"][rng.integers(0, 3)]
    log(f"random by-key seed={seed} n={n} {np.dtype(dt).name}/{np.dtype(vdt).name} runs={runs} op={op}")
    dk, dv = g.to_dev(keys), g.to_dev(vals)
    s = DeviceScan()
    so = g.empty(n, vdt)
    tmp = g.temp(DeviceScan.GetScanByKeyTempStorageBytes(np.dtype(dt).name, np.dtype(vdt).name, n))
    for inclusive in (False, True):
        (s.InclusiveSumByKey if inclusive else s.ExclusiveSumByKey)(tmp, dk, dv, so, n)
        assert (g.to_host(so) == o.scan_by_key(keys, vals, inclusive)).all(), inclusive
    uk, ag = g.empty(n, dt), g.empty(n, vdt)
    nr = torch.zeros(1, dtype=torch.int32, device="cuda")
    tmp = g.temp(DeviceReduce.GetReduceByKeyTempStorageBytes(np.dtype(dt).name, np.dtype(vdt).name, n))
    DeviceReduce().ReduceByKey(tmp, dk, dv, uk, ag, nr, op, n)
    rk, rv = o.reduce_by_key(keys, vals, {"sum": o.OP_SUM, "min": o.OP_MIN, "max": o.OP_MAX}[op])
    m = int(nr.item())
    assert m == rk.size and (g.to_host(uk)[:m] == rk).all() and (g.to_host(ag)[:m] == rv).all()


@pytest.mark.parametrize("seed,lr", cases(36))
def test_random_segments(gpu, seed, lr):
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceSegmentReduce

    rng, n, dt, kind = case_params(4000 + seed, lr)
    a = values(rng, dt, n, kind)
    S = max(1, int(rng.integers(1, 1 + max(1, n // int(rng.integers(1, 200))))))
    layout = seed % 3
    if layout < 2:  # tiling, in order or in a random order
        cuts = np.sort(rng.integers(0, n + 1, size=S - 1))
        bnd = np.concatenate([[0], cuts, [n]]).astype(np.uint32)
        b, e = bnd[:-1].copy(), bnd[1:].copy()
        if layout == 1:
            p = rng.permutation(S)
            b, e = b[p].copy(), e[p].copy()
    else:  # random windows: overlaps, gaps, inverted and empty ranges
        b = rng.integers(0, n + 1, size=S).astype(np.uint32)
        e = (b.astype(np.int64) + rng.integers(-5, 300, size=S)).clip(0, n).astype(np.uint32)
    log(f"random segments seed={seed} n={n} S={S} {np.dtype(dt).name} kind={kind} layout={layout}")
    d, db, de = g.to_dev(a), g.to_dev(b), g.to_dev(e)
    out, idx = g.empty(S, dt), g.empty(S, np.uint32)
    r = DeviceSegmentReduce()
    for nm, op in (("Sum", o.OP_SUM), ("Min", o.OP_MIN), ("Max", o.OP_MAX)):
        getattr(r, nm)(None, d, out, S, db, de)
        assert (g.to_host(out) == o.segment_reduce(op, a, b, e)).all(), nm
    for nm, is_max in (("ArgMin", False), ("ArgMax", True)):
        getattr(r, nm)(None, d, out, idx, S, db, de)
        ev, ei = o.segment_reduce_arg(is_max, a, b, e)
        assert (g.to_host(out) == ev).all() and (g.to_host(idx) == ei).all(), nm


@pytest.mark.parametrize("seed,lr", cases(24))
def test_random_misaligned_and_variants(gpu, seed, lr):
    """Pointers 0-3 elements off their 16-byte alignment (the element-wise
    load paths), transform reduce, scan-by-key with Min/Max/Sum and an
    initial value over 32- or 64-bit values, ReduceByKey with 64-bit values,
    fixed-size segments up to 20000 elements (the workgroup path)."""
    import torch

    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceReduce, DeviceScan, DeviceRadixSort, DeviceSegmentReduce

    rng, n, dt, kind = case_params(5000 + seed, lr)
    pad = int(rng.integers(0, 4))
    a = values(rng, dt, n, kind)
    ops = {"sum": o.OP_SUM, "min": o.OP_MIN, "max": o.OP_MAX}
    log(f"random misaligned seed={seed} n={n} {np.dtype(dt).name} kind={kind} pad={pad}")
    d = g.to_dev(a, pad=pad)
    out = g.empty(1, dt, pad=pad % 2)
    r = DeviceReduce()
    tmp = g.temp(DeviceReduce.GetTempStorageBytes(np.dtype(dt).name, n))
    r.Sum(tmp, d, out, n)
    assert g.to_host(out)[0] == o.reduce(o.OP_SUM, a)
    xf = ["identity", "negate", "abs", "square"][seed % 4]
    if np.dtype(dt).kind == "i" or xf in ("identity", "square"):
        op = ["sum", "min", "max"][seed % 3]
        r.TransformReduce(tmp, d, out, n, op, xf, 7)
        assert g.to_host(out)[0] == o.reduce_transform(ops[op], ["identity", "negate", "abs", "square"].index(xf), a, 7)
    so = g.empty(n, dt, pad=(pad + 1) % 4)
    tmp = g.temp(DeviceScan.GetTempStorageBytes(np.dtype(dt).name, n))
    DeviceScan().InclusiveSum(tmp, d, so, n)
    assert (g.to_host(so) == o.scan(a, True)).all()
    ko = g.empty(n, dt, pad=(pad + 2) % 4)
    tmp = g.temp(DeviceRadixSort.GetSortKeysTempStorageBytes(np.dtype(dt).name, n))
    DeviceRadixSort().SortKeysDescending(tmp, d, ko, n)
    assert (g.to_host(ko) == o.radix_sort(a, descending=True)).all()
    run = int(rng.integers(1, 300))
    keys = np.repeat(rng.integers(0, 4, size=n // run + 1), run)[:n].astype(dt)
    vdt = [np.int32, np.int64][seed % 2]
    vals = values(rng, vdt, n, 1)
    op = ["sum", "min", "max"][(seed // 2) % 3]
    dk, dv = g.to_dev(keys, pad=pad), g.to_dev(vals, pad=pad)
    sv = g.empty(n, vdt, pad=pad)
    tmp = g.temp(DeviceScan.GetScanByKeyTempStorageBytes(np.dtype(dt).name, np.dtype(vdt).name, n))
    DeviceScan().ExclusiveScanByKey(tmp, dk, dv, sv, op, n, -3)
    assert (g.to_host(sv) == o.scan_by_key(keys, vals, False, ops[op], -3)).all()
    uk, ag = g.empty(n, dt, pad=pad), g.empty(n, vdt, pad=pad)
    nr = torch.zeros(1, dtype=torch.int32, device="cuda")
    tmp = g.temp(DeviceReduce.GetReduceByKeyTempStorageBytes(np.dtype(dt).name, np.dtype(vdt).name, n))
    r.ReduceByKey(tmp, dk, dv, uk, ag, nr, op, n)
    rk, rv = o.reduce_by_key(keys, vals, ops[op])
    m = int(nr.item())
    assert m == rk.size and (g.to_host(uk)[:m] == rk).all() and (g.to_host(ag)[:m] == rv).all()
    size = min(n, int(np.exp(rng.uniform(0, np.log(20000)))))
    S = max(1, n // size)
    b, e = o.fixed_segments(S, size)
    sout, sidx = g.empty(S, dt, pad=pad), g.empty(S, np.uint32)
    DeviceSegmentReduce().Max(None, d, sout, S, size)
    assert (g.to_host(sout) == o.segment_reduce(o.OP_MAX, a, b, e)).all()
    DeviceSegmentReduce().ArgMin(None, d, sout, sidx, S, size)
    ev, ei = o.segment_reduce_arg(False, a, b, e)
    assert (g.to_host(sout) == ev).all() and (g.to_host(sidx) == ei).all()


@pytest.mark.parametrize("seed,lr", cases(24))
def test_random_floats(gpu, seed, lr):
    """float32 / float64 data (normal at a random scale, few distinct values,
    +-0, +-inf): sorts and Min/Max/Arg* exact against the oracle, sums and
    scans within 1e-5 * sum|x| of float64 (finite data)."""
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceReduce, DeviceScan, DeviceRadixSort, DeviceSegmentReduce

    rng, n, _, kind = case_params(6000 + seed, lr)
    dt = [np.float32, np.float64][seed % 2]
    if kind == 0:
        a = rng.standard_normal(n) * 10 ** rng.uniform(-3, 3)
    elif kind == 1:
        a = rng.integers(-3, 4, size=n).astype(np.float64) * 0.5
    elif kind == 2:
        a = rng.standard_normal(n)
        a[rng.random(n) < 0.05] = 0.0
        a[rng.random(n) < 0.05] = -0.0
    else:
        a = rng.standard_normal(n)
        a[rng.random(n) < 0.01] = np.inf
        a[rng.random(n) < 0.01] = -np.inf
    a = a.astype(dt)
    finite = kind != 3
    rt = 1e-5
    log(f"random floats seed={seed} n={n} {np.dtype(dt).name} kind={kind}")
    d = g.to_dev(a)
    out, idx = g.empty(1, dt), g.empty(1, np.uint32)
    r = DeviceReduce()
    tmp = g.temp(DeviceReduce.GetTempStorageBytes(np.dtype(dt).name, n))
    for nm, op in (("Min", o.OP_MIN), ("Max", o.OP_MAX)):
        getattr(r, nm)(tmp, d, out, n)
        assert g.to_host(out)[0] == o.reduce(op, a), nm
    if finite:
        r.Sum(tmp, d, out, n)
        s, ab = o.reduce_f64(a)
        assert abs(float(g.to_host(out)[0]) - s) <= rt * ab + 1e-30
    tmpa = g.temp(DeviceReduce.GetArgTempStorageBytes(np.dtype(dt).name, n))
    r.ArgMin(tmpa, d, out, idx, n)
    v, i = o.reduce_arg(False, a)
    assert g.to_host(out)[0] == v and g.to_host(idx)[0] == i
    if finite:
        so = g.empty(n, dt)
        tmps = g.temp(DeviceScan.GetTempStorageBytes(np.dtype(dt).name, n))
        DeviceScan().InclusiveSum(tmps, d, so, n)
        ref, ab = o.scan_f64(a, True)
        assert (np.abs(g.to_host(so).astype(np.float64) - ref) <= rt * ab + 1e-30).all()
    desc = bool(rng.integers(0, 2))
    ko, vo = g.empty(n, dt), g.empty(n, np.uint32)
    v = np.arange(n, dtype=np.uint32)
    tmp = g.temp(DeviceRadixSort.GetSortPairsTempStorageBytes(np.dtype(dt).name, "uint32", n))
    srt = DeviceRadixSort()
    (srt.SortPairsDescending if desc else srt.SortPairs)(tmp, d, ko, g.to_dev(v), vo, n)
    rk, rv = o.radix_sort(a, v, descending=desc)
    assert g.to_host(ko).tobytes() == rk.tobytes() and (g.to_host(vo) == rv).all()
    S = max(1, int(rng.integers(1, 1 + max(1, n // int(rng.integers(1, 200))))))
    cuts = np.sort(rng.integers(0, n + 1, size=S - 1))
    bnd = np.concatenate([[0], cuts, [n]]).astype(np.uint32)
    p = rng.permutation(S)
    b, e = bnd[:-1][p].copy(), bnd[1:][p].copy()
    db, de = g.to_dev(b), g.to_dev(e)
    sout, sidx = g.empty(S, dt), g.empty(S, np.uint32)
    seg = DeviceSegmentReduce()
    seg.Max(None, d, sout, S, db, de)
    assert (g.to_host(sout) == o.segment_reduce(o.OP_MAX, a, b, e)).all()
    seg.ArgMax(None, d, sout, sidx, S, db, de)
    ev, ei = o.segment_reduce_arg(True, a, b, e)
    assert (g.to_host(sout) == ev).all() and (g.to_host(sidx) == ei).all()
    if finite:
        seg.Sum(None, d, sout, S, db, de)
        s, ab = o.segment_reduce_f64(a, b, e)
        assert (np.abs(g.to_host(sout).astype(np.float64) - s) <= rt * ab + 1e-30).all()
