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


def test_flat_wave_ending_in_empty_segments_past_the_input(gpu):
    """A wave whose sorted segments tile the end of the input and whose last
    lanes are empty or inverted segments with begins past the input.  Only
    end <= begin makes a segment empty, so its begin may lie anywhere: the
    flat path must take its read window from the non-empty segments.  The
    input is a whole 16 MiB allocation (torch gives sizes of 10 MiB and more
    a segment of their own, rounded to 2 MiB), so a read past n would leave
    the mapping; n * 4 is a multiple of 16, so no 16-byte load straddles n."""
    import gpu_util as g
    import torch

    n = 4 << 20
    rng = np.random.default_rng(2024)
    T = 64 * 512 + 20  # the last wave: 20 tiling segments, then 44 empty ones
    cuts = np.sort(rng.choice(np.arange(1, n), T - 1, replace=False)).astype(np.int64)
    b = np.concatenate([[0], cuts]).astype(np.uint32)
    e = np.concatenate([cuts, [n]]).astype(np.uint32)
    eb = (n + 7 * np.arange(44)).astype(np.uint32)
    ee = eb.copy()
    ee[1::2] = eb[1::2] // 2  # inverted: end < begin
    b, e = np.concatenate([b, eb]), np.concatenate([e, ee])
    S = b.size
    log(f"segment flat wave ending past the input n={n} S={S}")
    for dtype in (np.int32, np.float32):
        a = g.random_array(dtype, n, seed=11)
        d = torch.empty(n, dtype=g._NP2T[np.dtype(dtype)], device="cuda")  # exactly 16 MiB
        d.copy_(torch.from_numpy(a))
        got = seg_call("Sum", d, S, (b, e), dtype)
        if dtype == np.int32:
            assert same(got, o.segment_reduce(o.OP_SUM, a, b, e))
        else:
            s, ab = o.segment_reduce_f64(a, b, e)
            assert (np.abs(got.astype(np.float64) - s) <= RTOL_SEG * ab + 1e-30).all()
        assert same(seg_call("Max", d, S, (b, e), dtype), o.segment_reduce(o.OP_MAX, a, b, e))
        v, i = seg_call("ArgMin", d, S, (b, e), dtype, arg=True)
        ev, ei = o.segment_reduce_arg(False, a, b, e)
        assert same(v, ev) and (i == ei).all()


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


# ------------------------------------------------------------------ Reduce / Min / Max / Arg*, CSR and fixed-size
ALL_DTYPES = [np.int32, np.uint32, np.float32, np.int64, np.uint64, np.float64]
SHUFFLED_1024 = "segment_shuffled_1024_i32.bin"


def same(got, ref) -> bool:
    """Integers bit-exact; floats equal in value (Min/Max of -0.0 and +0.0
    return either zero depending on the fold order)."""
    if got.dtype.kind == "f":
        return bool(np.array_equal(got, ref))
    return got.tobytes() == ref.tobytes()


def seg_call(method, d_in, S, offsets, dtype, *extra, arg=False):
    """Runs DeviceSegmentReduce.<method>; offsets = (begin, end) host arrays or (segment_size,)."""
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceSegmentReduce

    out = g.empty(S, dtype)
    idx = g.empty(S, np.uint32) if arg else None
    off = offsets if isinstance(offsets[0], int) else (g.to_dev(offsets[0]), g.to_dev(offsets[1]))
    r = DeviceSegmentReduce()
    if arg:
        getattr(r, method)(None, d_in, out, idx, S, *off)
        return g.to_host(out), g.to_host(idx)
    getattr(r, method)(None, d_in, out, S, *off, *extra)
    return g.to_host(out)


def test_kat_fixed_sum(gpu):
    # device_segment_reduce.cpp fixed_segment_reduce: 0..1023 in fixed segments of 32
    import gpu_util as g

    got = seg_call("Sum", g.to_dev(np.arange(1024, dtype=np.int32)), 32, (32,), np.int32)
    assert (got == np.array([32 * 32 * i + 496 for i in range(32)])).all()


def test_kat_argmax_csr_and_fixed_argmin(gpu):
    # device_segment_reduce.cpp segment_reduce_arg_max (11 segments of <= 100) and
    # fixed_segment_reduce_arg_min (fixed 32) over the shuffled 0..1023
    import gpu_util as g

    a = golden(SHUFFLED_1024, np.int32)
    d = g.to_dev(a)
    b = np.arange(0, 1024, 100, dtype=np.uint32)
    e = np.minimum(b + 100, 1024).astype(np.uint32)
    v, i = seg_call("ArgMax", d, 11, (b, e), np.int32, arg=True)
    assert (v == np.array([a[x:y].max() for x, y in zip(b, e)])).all()
    assert (i == np.array([a[x:y].argmax() for x, y in zip(b, e)])).all()
    v, i = seg_call("ArgMin", d, 32, (32,), np.int32, arg=True)
    assert (v == a.reshape(32, 32).min(axis=1)).all() and (i == a.reshape(32, 32).argmin(axis=1)).all()
    v2, i2 = seg_call("Argmin", d, 11, (b, e), np.int32, arg=True)  # the reference's CSR spelling
    assert (v2 == np.array([a[x:y].min() for x, y in zip(b, e)])).all()


@pytest.mark.parametrize("dtype", ALL_DTYPES)
@pytest.mark.parametrize("op", ["min", "max", "sum"])
def test_reduce_init_csr_vs_oracle(gpu, dtype, op):
    import gpu_util as g

    n, S = 400_000, 6000
    b, e = o.segments(21, 22, n, S)
    e[::17] = b[::17]  # extra empty segments
    dt = np.dtype(dtype)
    a = g.random_array(dtype, n, seed=23)
    if dt.kind == "f" and op == "sum":
        a = np.round(a).astype(dt)  # integral values: float sums exact in any order
    init = dt.type(a[7])
    log(f"segment Reduce {op} {dt.name}")
    got = seg_call("Reduce", g.to_dev(a), S, (b, e), dtype, op, init)
    ref = o.segment_reduce({"sum": o.OP_SUM, "min": o.OP_MIN, "max": o.OP_MAX}[op], a, b, e, init=init)
    assert same(got, ref)
    if op != "sum":
        got = seg_call(op.capitalize(), g.to_dev(a), S, (b, e), dtype)
        assert same(got, o.segment_reduce({"min": o.OP_MIN, "max": o.OP_MAX}[op], a, b, e))


@pytest.mark.parametrize("size", [0, 1, 7, 64, 100, 513, 8192, 8193, 20_000])
@pytest.mark.parametrize("dtype", [np.int32, np.float64])
def test_fixed_size_all_ops_vs_oracle(gpu, size, dtype):
    import gpu_util as g

    S = 600 if size <= 8192 else 150
    n = max(S * size, 1)
    dt = np.dtype(dtype)
    a = g.random_array(dtype, n, seed=size)
    if dt.kind == "f":
        a = np.round(a).astype(dt)
    d = g.to_dev(a)
    b, e = o.fixed_segments(S, size)
    log(f"segment fixed size={size} {dt.name}")
    for method, op in (("Sum", o.OP_SUM), ("Min", o.OP_MIN), ("Max", o.OP_MAX)):
        assert same(seg_call(method, d, S, (size,), dtype), o.segment_reduce(op, a, b, e)), method
    for method, is_max in (("ArgMin", False), ("ArgMax", True)):
        v, i = seg_call(method, d, S, (size,), dtype, arg=True)
        ev, ei = o.segment_reduce_arg(is_max, a, b, e)
        assert same(v, ev) and (i == ei).all(), method


@pytest.mark.parametrize("dtype", ALL_DTYPES)
def test_arg_csr_ties_empty_long(gpu, dtype):
    import gpu_util as g

    rng = np.random.default_rng(31)
    n, S = 1 << 20, 2500
    b = rng.integers(0, n, S).astype(np.uint32)
    L = rng.integers(0, 400, S)
    L[::40] = rng.integers(8193, 60_000, L[::40].size)  # long -> workgroup path
    L[::9] = 0
    e = np.minimum(b.astype(np.int64) + L, n).astype(np.uint32)
    e[::13] = b[::13] // 2  # inverted -> empty
    a = rng.integers(0, 50, n).astype(dtype)  # many ties
    d = g.to_dev(a)
    for method, is_max in (("ArgMin", False), ("ArgMax", True)):
        log(f"segment {method} {np.dtype(dtype).name}")
        v, i = seg_call(method, d, S, (b, e), dtype, arg=True)
        ev, ei = o.segment_reduce_arg(is_max, a, b, e)
        assert same(v, ev) and (i == ei).all()


def test_arg_infinite_and_all_equal(gpu):
    import gpu_util as g

    a = np.array([-np.inf, -np.inf, np.inf, np.inf, 3, 3, 3], np.float32)
    b, e = np.array([0, 2, 4, 7], np.uint32), np.array([2, 4, 7, 7], np.uint32)
    d = g.to_dev(a)
    v, i = seg_call("ArgMax", d, 4, (b, e), np.float32, arg=True)
    assert list(i) == [1, 1, 2, 1] and v[0] == -np.inf and v[1] == np.inf and v[3] == np.finfo(np.float32).min
    v, i = seg_call("ArgMin", d, 4, (b, e), np.float32, arg=True)
    assert list(i) == [0, 0, 0, 1] and v[3] == np.finfo(np.float32).max


def contiguous_layout(lengths):
    """CSR begin/end offsets of segments that tile [0, sum(lengths)) in order."""
    L = np.asarray(lengths, dtype=np.int64)
    e = np.cumsum(L)
    b = e - L
    return b.astype(np.uint32), e.astype(np.uint32)


# Segments that tile one range take the flat path of a wave (64 segments):
# chunk-sized, lane-sized and single-element segments, empty segments at the
# start, middle and end of a wave, a wave of empty segments only, the longest
# flat segment (8192) and a long one (8193, whose wave falls back).
FLAT_LAYOUTS = {
    "lane_and_chunk": [16, 1024, 1, 15, 17, 1023, 1025, 512, 513, 2, 3, 4] * 11,
    "empty_edges": [0, 0, 5, 0, 0, 130, 0, 7, 0, 0] * 13 + [0] * 70 + [9, 0, 0],
    "all_empty_wave": [3] * 64 + [0] * 64 + [4] * 70,
    "max_flat_and_long": [8192, 1, 8192, 0, 100] + [70] * 59 + [8193, 5, 0, 6] + [128] * 60,
}


@pytest.mark.parametrize("layout", sorted(FLAT_LAYOUTS))
@pytest.mark.parametrize("dtype", [np.int32, np.int64])
@pytest.mark.parametrize("pad", [0, 1])
def test_contiguous_layouts_sum(gpu, layout, dtype, pad):
    import gpu_util as g

    b, e = contiguous_layout(FLAT_LAYOUTS[layout])
    n = int(e[-1])
    a = g.random_array(dtype, n, seed=n + pad)
    log(f"segment contiguous {layout} {np.dtype(dtype).name} pad={pad}")
    d = g.to_dev(a, pad=pad)  # pad = 1: misaligned input takes the segment-walking path
    assert (run(d, b, e, dtype) == o.segment_reduce(o.OP_SUM, a, b, e)).all()


@pytest.mark.parametrize("layout", sorted(FLAT_LAYOUTS))
@pytest.mark.parametrize("dtype", [np.int32, np.float32, np.uint64, np.float64])
def test_contiguous_layouts_min_max_arg(gpu, layout, dtype):
    import gpu_util as g

    b, e = contiguous_layout(FLAT_LAYOUTS[layout])
    n = int(e[-1])
    rng = np.random.default_rng(n)
    a = rng.integers(0, 40, n).astype(dtype)  # ties
    d = g.to_dev(a)
    S = b.size
    log(f"segment contiguous min/max/arg {layout} {np.dtype(dtype).name}")
    for method, op in (("Min", o.OP_MIN), ("Max", o.OP_MAX)):
        assert same(seg_call(method, d, S, (b, e), dtype), o.segment_reduce(op, a, b, e))
    for method, is_max in (("ArgMin", False), ("ArgMax", True)):
        v, i = seg_call(method, d, S, (b, e), dtype, arg=True)
        ev, ei = o.segment_reduce_arg(is_max, a, b, e)
        assert same(v, ev) and (i == ei).all()


def test_contiguous_then_scattered_waves(gpu):
    """Waves of one launch take different paths: tiling waves, then waves with
    gaps and overlaps."""
    import gpu_util as g

    rng = np.random.default_rng(77)
    b1, e1 = contiguous_layout(rng.geometric(1 / 100, 256 * 3) - 1)
    n = int(e1[-1]) + 50_000
    b2 = rng.integers(0, n - 300, 256 * 2).astype(np.uint32)
    e2 = (b2 + rng.integers(0, 300, b2.size)).astype(np.uint32)
    b, e = np.concatenate([b1, b2]), np.concatenate([e1, e2])
    a = g.random_array(np.int32, n, seed=5)
    assert (run(g.to_dev(a), b, e, np.int32) == o.segment_reduce(o.OP_SUM, a, b, e)).all()


# ------------------------------------------------------------------ layouts that do not tile one range
def gapped_layout(lengths, gaps):
    """Sorted, disjoint CSR ranges: segment i is followed by gaps[i] elements
    that belong to no segment."""
    L = np.asarray(lengths, dtype=np.int64)
    G = np.asarray(gaps, dtype=np.int64)
    b = np.concatenate([[0], np.cumsum(L + G)[:-1]])
    return b.astype(np.uint32), (b + L).astype(np.uint32)


def _nontiling_layouts():
    rng = np.random.default_rng(123)
    geo = rng.geometric(1 / 100, 1500) - 1  # mean ~99, ~1 % empty
    short = rng.integers(0, 4, 3000)  # several ends per 64-element window
    tb, te = contiguous_layout(geo)
    perm = rng.permutation(geo.size)
    sb, se = contiguous_layout(short)
    sperm = rng.permutation(short.size)
    lay = {
        # sorted with gaps: the contiguous path reads the gaps and drops them
        "gaps_one": gapped_layout(geo, np.ones(geo.size, np.int64)),
        "gaps_mixed": gapped_layout(geo, rng.integers(0, 40, geo.size) * (rng.random(geo.size) < 0.3)),
        # gaps holding more elements than the segments: gather
        "gaps_too_wide": gapped_layout(rng.integers(0, 10, 900), np.full(900, 200)),
        # not sorted: gather
        "permuted": (tb[perm], te[perm]),
        "short_permuted": (sb[sperm], se[sperm]),
        "descending": (tb[::-1].copy(), te[::-1].copy()),
    }
    # sorted and overlapping (sliding windows of 1..300 elements, stride 50)
    ob = (np.arange(2000, dtype=np.int64) * 50).astype(np.uint32)
    lay["sliding_windows"] = (ob, (ob + rng.integers(1, 300, ob.size)).astype(np.uint32))
    # sorted and disjoint, with inverted ranges (end < begin: empty) between them
    ib, ie = gapped_layout(geo, rng.integers(0, 3, geo.size))
    ie = ie.copy()
    ie[::10] = ib[::10] - np.minimum(ib[::10], 5)
    lay["gaps_inverted_empty"] = (ib, ie)
    return lay


NONTILING = _nontiling_layouts()


@pytest.mark.parametrize("layout", sorted(NONTILING))
@pytest.mark.parametrize("dtype", [np.int32, np.float32, np.int64, np.float64])
@pytest.mark.parametrize("pad", [0, 1])
def test_nontiling_layouts_all_ops(gpu, layout, dtype, pad):
    import gpu_util as g

    b, e = NONTILING[layout]
    n = int(max(e.max(), b.max())) + 7
    rng = np.random.default_rng(n + pad)
    a = rng.integers(-40, 40, n).astype(dtype)  # ties; float sums of small integers are exact in any order
    d = g.to_dev(a, pad=pad)  # pad = 1: 16-byte loads are off, every wave gathers
    S = b.size
    log(f"segment nontiling {layout} {np.dtype(dtype).name} pad={pad}")
    for method, op in (("Sum", o.OP_SUM), ("Min", o.OP_MIN), ("Max", o.OP_MAX)):
        assert same(seg_call(method, d, S, (b, e), dtype), o.segment_reduce(op, a, b, e)), method
    for method, is_max in (("ArgMin", False), ("ArgMax", True)):
        v, i = seg_call(method, d, S, (b, e), dtype, arg=True)
        ev, ei = o.segment_reduce_arg(is_max, a, b, e)
        assert same(v, ev) and (i == ei).all(), method


def test_nontiling_full_size_permuted(gpu):
    """C5's segments in a random order (every wave gathers) at full size:
    Sum within the float64 bound, ArgMax exact."""
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n, S = 1 << 27, 1 << 20
    log("segment f32 full 2^27 / 2^20 permuted")
    d = datagen.normal_f32(n, seed=datagen.SEED_SEG_VALUES)
    b, e = datagen.segments(n, S)
    perm = np.random.default_rng(3).permutation(S)
    b, e = b[perm].copy(), e[perm].copy()
    got = run(d, b, e, np.float32)
    h = g.to_host(d)
    s, ab = o.segment_reduce_f64(h, b, e)
    assert (np.abs(got.astype(np.float64) - s) <= RTOL_SEG * ab).all()
    v, i = seg_call("ArgMax", d, S, (b, e), np.float32, arg=True)
    ev, ei = o.segment_reduce_arg(True, h, b, e)
    assert same(v, ev) and (i == ei).all()


@pytest.mark.parametrize("layout", ["reversed_waves", "random_tiny"])
def test_gather_lowest_segment_late_in_wave(gpu, layout):
    """Gather waves whose lowest-addressed segments sit late in the wave's
    virtual range, so an element's byte offset from the wave's lowest
    begin is smaller than its position in the gathered order: every wave of
    "reversed_waves" (64 segments of 1-3 elements laid out in descending
    address order, 2^22 segments), and the layout that exposed a load whose
    offset had been split between a wrapped VGPR part and an immediate
    (tiling segments of mean length ~1.4 in a random order, the values one
    constant).  Every op, exact against the oracle, the output's guard
    region untouched."""
    import torch

    import gpu_util as g

    rng = np.random.default_rng(17 if layout == "reversed_waves" else 23)
    if layout == "reversed_waves":
        S = 1 << 22
        lens = rng.integers(1, 4, size=S).astype(np.int64)
        w = lens.reshape(-1, 64)
        # within each wave, lane k's segment lies after lane k + 1's
        starts = np.cumsum(w[:, ::-1], axis=1) - w[:, ::-1]
        wave_base = np.concatenate([[0], np.cumsum(w.sum(axis=1))[:-1]])
        b = (wave_base[:, None] + starts[:, ::-1]).ravel()
        e = b + lens
        n = int(e.max())
        a = rng.integers(-(1 << 30), 1 << 30, size=n, dtype=np.int32)
    else:
        n, S = 6_000_007, 4_200_011
        cuts = np.sort(rng.integers(0, n + 1, size=S - 1))
        bnd = np.concatenate([[0], cuts, [n]])
        perm = rng.permutation(S)
        b, e = bnd[:-1][perm], bnd[1:][perm]
        a = np.full(n, -1201695826, dtype=np.int32)
    b, e = b.astype(np.uint32), e.astype(np.uint32)
    log(f"segment gather, lowest segment late: {layout} n={n} S={S}")
    d, db, de = g.to_dev(a), g.to_dev(b), g.to_dev(e)
    from lc_parallel_primitive_amd import DeviceSegmentReduce

    r = DeviceSegmentReduce()
    outg = torch.full((S + 1024,), 7, dtype=torch.int32, device="cuda")
    idxg = torch.full((S + 1024,), 7, dtype=torch.int32, device="cuda")
    out, idx = outg[:S], idxg[:S].view(torch.uint32)
    for method, op in (("Sum", o.OP_SUM), ("Min", o.OP_MIN), ("Max", o.OP_MAX)):
        getattr(r, method)(None, d, out, S, db, de)
        assert (g.to_host(out) == o.segment_reduce(op, a, b, e)).all(), method
    for method, is_max in (("ArgMin", False), ("ArgMax", True)):
        getattr(r, method)(None, d, out, idx, S, db, de)
        ev, ei = o.segment_reduce_arg(is_max, a, b, e)
        assert (g.to_host(out) == ev).all() and (g.to_host(idx) == ei).all(), method
    assert (g.to_host(outg[S:]) == 7).all() and (g.to_host(idxg[S:]) == 7).all()


def test_segments_more_than_4gib_apart(gpu):
    """A wave whose segments lie more than 4 GiB apart (int32 input of 2^30 +
    2^20 elements, value = index) takes the one-segment-at-a-time path:
    results from closed forms."""
    import torch

    import gpu_util as g

    n = (1 << 30) + (1 << 20)
    log("segment int32 2^30+2^20 segments > 4 GiB apart")
    d = torch.arange(n, dtype=torch.int32, device="cuda")
    S = 200
    rng = np.random.default_rng(8)
    L = rng.integers(0, 300, S)
    L[5] = 0
    L[17] = 9000  # long: workgroup path
    b = np.where(np.arange(S) % 2 == 0, np.arange(S) * 400, n - 20_000 + np.arange(S) * 90).astype(np.int64)
    e = np.minimum(b + L, n)
    bu, eu = b.astype(np.uint32), e.astype(np.uint32)
    sums = [(int((x + y - 1) * (y - x) // 2)) if y > x else 0 for x, y in zip(b, e)]
    expect_sum = np.array([(v + 2**31) % 2**32 - 2**31 for v in sums], dtype=np.int64).astype(np.int32)
    assert (seg_call("Sum", d, S, (bu, eu), np.int32) == expect_sum).all()
    empty = e <= b
    mn = seg_call("Min", d, S, (bu, eu), np.int32)
    assert (mn[~empty] == b[~empty]).all() and (mn[empty] == np.iinfo(np.int32).max).all()
    v, i = seg_call("ArgMax", d, S, (bu, eu), np.int32, arg=True)
    assert (v[~empty] == e[~empty] - 1).all() and (i[~empty] == (e - b - 1)[~empty]).all()
    assert (i[empty] == 1).all()


def test_segments_spanning_2_to_4_gib(gpu):
    """Waves whose segments span 2-4 GiB of input (an int32 input of 3 * 2^28
    elements, value = index): more than one buffer resource covers (offsets
    would pass 2^31), so they fold one segment at a time; the
    lowest-addressed segment of each wave comes last in it.  Results from
    closed forms."""
    import torch

    n = 3 << 28
    log("segment int32 3*2^28 gather spans 2-4 GiB")
    d = torch.arange(n, dtype=torch.int32, device="cuda")
    S = 256
    rng = np.random.default_rng(12)
    L = rng.integers(0, 200, S)
    L[9] = 0
    i = np.arange(S)
    # even lanes near the end of the input, odd lanes near its start in
    # descending order (the wave's lowest begin is its last odd lane)
    b = np.where(i % 2 == 0, n - 40_000 + i * 100, (S - i) * 300).astype(np.int64)
    e = np.minimum(b + L, n)
    bu, eu = b.astype(np.uint32), e.astype(np.uint32)
    sums = [(int((x + y - 1) * (y - x) // 2)) if y > x else 0 for x, y in zip(b, e)]
    expect_sum = np.array([(v + 2**31) % 2**32 - 2**31 for v in sums], dtype=np.int64).astype(np.int32)
    assert (seg_call("Sum", d, S, (bu, eu), np.int32) == expect_sum).all()
    empty = e <= b
    mx = seg_call("Max", d, S, (bu, eu), np.int32)
    assert (mx[~empty] == e[~empty] - 1).all() and (mx[empty] == np.iinfo(np.int32).min).all()
    v, ix = seg_call("ArgMin", d, S, (bu, eu), np.int32, arg=True)
    assert (v[~empty] == b[~empty]).all() and (ix[~empty] == 0).all() and (ix[empty] == 1).all()


def test_segments_at_the_top_of_the_32_bit_range(gpu):
    """Segments ending at element 2^32 - 1 (an int32 input of 2^32 - 1
    elements, 16 GiB): a tiling layout there is past the contiguous path's
    range limit and gathers; element indices near 2^32 must not wrap.  Values
    are 1 except a few marked elements, so sums are lengths plus marks and
    ArgMax finds the marks."""
    import torch

    n = (1 << 32) - 1
    log("segment int32 2^32-1 elements, segments at the top")
    d = torch.ones(n, dtype=torch.int32, device="cuda")
    rng = np.random.default_rng(12)
    L = rng.integers(0, 200, 300)
    L[7] = 0
    e_last = n
    e = e_last - np.concatenate([[0], np.cumsum(L[::-1])[:-1]])[::-1]
    b = e - L
    b, e = b.astype(np.int64), e.astype(np.int64)
    marks = {int(b[i] + L[i] // 2): 1000 + i for i in range(0, 300, 5) if L[i] > 0}
    marks[n - 1] = 7777  # the very last element
    for pos, v in marks.items():
        d[pos] = v
    bu, eu = b.astype(np.uint32), e.astype(np.uint32)
    S = b.size
    want = L.astype(np.int64).copy()
    for s_ in range(S):
        for pos, v in marks.items():
            if b[s_] <= pos < e[s_]:
                want[s_] += v - 1
    assert (seg_call("Sum", d, S, (bu, eu), np.int32) == want.astype(np.int32)).all()
    v, i = seg_call("ArgMax", d, S, (bu, eu), np.int32, arg=True)
    for s_ in range(S):
        ms = [(val, pos) for pos, val in marks.items() if b[s_] <= pos < e[s_]]
        if ms:
            val, pos = max(ms)
            assert v[s_] == val and i[s_] == pos - b[s_]
        elif L[s_] > 0:
            assert v[s_] == 1 and i[s_] == L[s_] - 1  # ties: the largest index
    del d
    torch.cuda.empty_cache()


def _mixed_layout(rng, n):
    """Blocks of whole waves (64 segments), each of one kind: tiling, gapped,
    permuted, overlapping, long (> 8192) or empty segments, over [0, n)."""
    bs, es = [], []
    kinds = ["tiling", "gaps", "permuted", "overlap", "long", "empty"]
    pos = 0
    for _ in range(int(rng.integers(6, 14))):
        kind = kinds[int(rng.integers(0, len(kinds)))]
        m = 64 * int(rng.integers(1, 4)) - int(rng.integers(0, 2)) * int(rng.integers(1, 63))  # >= 2
        if kind == "long":
            L = rng.integers(8193, 20000, m)
        elif kind == "empty":
            L = np.zeros(m, np.int64)
        else:
            L = rng.geometric(1 / 60, m) - 1
        if kind in ("tiling", "permuted", "long", "empty"):
            e = pos + np.cumsum(L)
            b = e - L
        elif kind == "gaps":
            g = rng.integers(0, 30, m) * (rng.random(m) < 0.5)
            e = pos + np.cumsum(L + g)
            b = e - L
        else:  # overlapping: begins every 20 elements
            b = pos + np.arange(m, dtype=np.int64) * 20
            e = b + L
        if kind == "permuted":
            p = rng.permutation(m)
            b, e = b[p], e[p]
        if int(e.max()) > n or int(b.max()) > n:
            continue  # does not fit: try another block
        pos = int(max(e.max(), b.max()))
        bs.append(b)
        es.append(e)
    if not bs:
        e = np.cumsum(rng.geometric(1 / 60, 64) - 1)
        bs, es = [e - (e - np.concatenate([[0], e[:-1]]))], [e]
    return np.concatenate(bs).astype(np.uint32), np.concatenate(es).astype(np.uint32)


@pytest.mark.parametrize("seed", range(12))
def test_mixed_layouts_random(gpu, seed):
    """Random mixes of layouts in one launch (waves of different paths side by
    side, ragged last wave), every op, against the oracle."""
    import gpu_util as g

    rng = np.random.default_rng(9000 + seed)
    dtype = [np.int32, np.float32, np.int64, np.float64, np.uint32, np.uint64][seed % 6]
    n = 1_500_000
    b, e = _mixed_layout(rng, n)
    a = rng.integers(0, 50, n).astype(dtype)  # ties; exact float sums
    d = g.to_dev(a, pad=seed % 2)
    S = b.size
    log(f"segment mixed layouts seed={seed} S={S} {np.dtype(dtype).name}")
    for method, op in (("Sum", o.OP_SUM), ("Min", o.OP_MIN), ("Max", o.OP_MAX)):
        assert same(seg_call(method, d, S, (b, e), dtype), o.segment_reduce(op, a, b, e)), method
    for method, is_max in (("ArgMin", False), ("ArgMax", True)):
        v, i = seg_call(method, d, S, (b, e), dtype, arg=True)
        ev, ei = o.segment_reduce_arg(is_max, a, b, e)
        assert same(v, ev) and (i == ei).all(), method
