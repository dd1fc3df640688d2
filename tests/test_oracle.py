"""Pins the CPU oracle (oracle/lcpp_oracle.c) before it is trusted as the
parity checker.  Each oracle function is checked against something it does
not share code with: the reference tests' known answers (golden fixtures
regenerated with libstdc++), numpy/Python library routines, closed forms,
published test vectors, and planted mistakes that must be caught."""
import ctypes

import numpy as np
import pytest

from conftest import golden
from oracle import oracle as o

SORT_DTYPES = [np.uint32, np.int32, np.float32, np.uint64, np.int64, np.float64]


# ------------------------------------------------------------------ generators
def test_splitmix64_published_vector():
    # Vigna's splitmix64.c, state 1234567: first five outputs
    st = ctypes.c_uint64(1234567)
    got = [o.lib().lcor_splitmix64_next(ctypes.byref(st)) for _ in range(5)]
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                   4593380528125082431, 16408922859458223821]


def test_counter_based_word_equals_sequential_stream():
    st = ctypes.c_uint64(99)
    seq = [o.lib().lcor_splitmix64_next(ctypes.byref(st)) for _ in range(100)]
    assert [o.word(99, i) for i in range(100)] == seq


def test_generators_ranges_and_distributions():
    a = o.gen("reduce_i32", 1 << 20, 0xC1)
    assert a.min() == -1000 and a.max() == 1000 and abs(a.mean()) < 2
    b = o.gen("u8_u32", 1 << 20, 0xC2A)
    assert b.min() == 0 and b.max() == 255
    c = o.gen("normal_f32", 1 << 20, 0xC2B)
    assert abs(c.mean()) < 0.01 and abs(c.std() - 1) < 0.01
    d = o.gen("keys_u32_and3", 1 << 20, 1, 2, 3)
    assert abs((d >> 24 == 0).mean() - (7 / 8) ** 8) < 0.01  # top digit 0 with p = 0.344
    e = o.gen("keys_u64_low16", 1 << 16, 4)
    assert (e >> 16 == 0).all()
    w = o.words(0xC1, 5)
    ex = ((w >> 32) * 2001 >> 32).astype(np.int64) - 1000
    assert (a[:5] == ex).all()


def test_segments_generator():
    b, e = o.segments(0xC5E, 0xC5F, 1 << 20, 1 << 13)
    L = e.astype(np.int64) - b
    assert b[0] == 0 and e[-1] == 1 << 20 and (b[1:] == e[:-1]).all() and (L >= 0).all()
    assert 0.03 < (L == 0).mean() < 0.07 and 110 < L.mean() < 150


# ------------------------------------------------------------------ reduce
def test_reduce_kat_ones():
    # device_reduce_test.cpp:66-90: Sum of N ones == N, N = 2^k + 1
    for k in range(0, 16):
        n = (1 << k) + 1
        assert o.reduce(o.OP_SUM, np.ones(n, np.uint32)) == n


def test_reduce_kat_min_max_shuffled():
    a = golden("reduce_shuffled_4096_i32.bin", np.int32)
    exp = golden("reduce_shuffled_4096_expect_min_max_sum_i32.bin", np.int32)
    assert o.reduce(o.OP_MIN, a) == exp[0] == 0
    assert o.reduce(o.OP_MAX, a) == exp[1] == 4095
    assert o.reduce(o.OP_SUM, a) == exp[2]


@pytest.mark.parametrize("dt", [np.int32, np.uint32, np.int64, np.uint64])
def test_reduce_integer_closed_form(dt):
    rng = np.random.default_rng(1)
    info = np.iinfo(dt)
    a = rng.integers(info.min, info.max, size=100_003, dtype=dt, endpoint=True)
    bits = 8 * a.itemsize
    exact = sum(int(x) for x in a) % (1 << bits)  # Python big ints, then wrap
    got = int(o.reduce(o.OP_SUM, a)) % (1 << bits)
    assert got == exact
    assert o.reduce(o.OP_MIN, a) == a.min() and o.reduce(o.OP_MAX, a) == a.max()
    assert o.reduce(o.OP_SUM, a, nthreads=5) == o.reduce(o.OP_SUM, a)


def test_reduce_empty_gives_init():
    assert o.reduce(o.OP_SUM, np.zeros(0, np.int32)) == 0
    assert o.reduce(o.OP_MIN, np.zeros(0, np.int32)) == np.iinfo(np.int32).max
    assert o.reduce(o.OP_MAX, np.zeros(0, np.float32)) == np.finfo(np.float32).min  # lowest()


def test_reduce_f64_against_fsum():
    import math

    a = o.gen("normal_f32", 200_001, 7)
    s, ab = o.reduce_f64(a)
    assert s == pytest.approx(math.fsum(float(x) for x in a), abs=1e-9)
    assert ab == pytest.approx(float(np.abs(a.astype(np.float64)).sum()), rel=1e-12)


def last_argmax(a: np.ndarray) -> int:
    """Index of the last maximum (ArgMaxOp breaks ties to the larger index)."""
    return a.size - 1 - int(np.argmax(a[::-1]))


@pytest.mark.parametrize("dt", SORT_DTYPES)
def test_reduce_arg_vs_numpy(dt):
    rng = np.random.default_rng(21)
    n = 60_007
    if np.issubdtype(dt, np.floating):
        a = rng.integers(-50, 50, size=n).astype(dt)  # many ties
    else:
        info = np.iinfo(dt)
        a = rng.integers(max(info.min, -50), 50, size=n, endpoint=True).astype(dt)
    v, i = o.reduce_arg(False, a)
    assert i == int(np.argmin(a)) and v == a.min()  # first occurrence
    v, i = o.reduce_arg(True, a)
    assert i == last_argmax(a) and v == a.max()  # last occurrence
    assert last_argmax(np.array([1, 3, 2, 3], dt)) == 3


def test_reduce_arg_kat_shuffled():
    # device_reduce_test.cpp:169-225: shuffled 0..4095, std::min/max_element
    a = golden("reduce_shuffled_4096_i32.bin", np.int32)
    assert o.reduce_arg(False, a) == (0, int(np.nonzero(a == 0)[0][0]))
    assert o.reduce_arg(True, a) == (4095, int(np.nonzero(a == 4095)[0][0]))


def test_reduce_arg_empty():
    assert o.reduce_arg(False, np.zeros(0, np.int32)) == (np.iinfo(np.int32).max, 0xFFFFFFFF)
    assert o.reduce_arg(True, np.zeros(0, np.float32)) == (np.finfo(np.float32).min, 0)


NP_XF = {o.XF_IDENTITY: lambda a: a, o.XF_NEGATE: np.negative, o.XF_ABS: np.abs,
         o.XF_SQUARE: lambda a: np.multiply(a, a)}
NP_OP = {o.OP_SUM: np.sum, o.OP_MIN: np.min, o.OP_MAX: np.max}


@pytest.mark.parametrize("dt", [np.int32, np.uint32, np.int64, np.uint64])
@pytest.mark.parametrize("xf", [o.XF_IDENTITY, o.XF_NEGATE, o.XF_ABS, o.XF_SQUARE])
@pytest.mark.parametrize("op", [o.OP_SUM, o.OP_MIN, o.OP_MAX])
def test_reduce_transform_integers_vs_numpy(dt, xf, op):
    rng = np.random.default_rng(xf * 3 + op)
    info = np.iinfo(dt)
    a = rng.integers(info.min, info.max, size=20_011, dtype=dt, endpoint=True)
    with np.errstate(over="ignore"):
        t = NP_XF[xf](a).astype(dt)  # element-type wraparound
        red = NP_OP[op](t, dtype=dt) if op == o.OP_SUM else NP_OP[op](t)
        init = dt(7)
        exp = NP_OP[op](np.array([init, red], dtype=dt), dtype=dt) if op == o.OP_SUM else NP_OP[op]([init, red])
    assert o.reduce_transform(op, xf, a, init) == exp


def test_reduce_transform_kat_max_of_squares():
    # device_reduce_test.cpp:92-117: max over shuffled 0..4095 of x*x, init 0 -> 4095^2
    a = golden("reduce_shuffled_4096_i32.bin", np.int32)
    assert o.reduce_transform(o.OP_MAX, o.XF_SQUARE, a, 0) == 4095 * 4095


# ------------------------------------------------------------------ scan
def test_scan_kat_ones():
    # device_scan_test.cpp:67-108: ones -> exclusive i, inclusive i+1
    for k in range(0, 16, 3):
        n = 1 << k
        x = np.ones(n, np.uint32)
        assert (o.scan(x, False) == np.arange(n, dtype=np.uint32)).all()
        assert (o.scan(x, True) == np.arange(1, n + 1, dtype=np.uint32)).all()


@pytest.mark.parametrize("dt", [np.int32, np.uint32, np.int64, np.uint64])
def test_scan_wraparound_vs_numpy(dt):
    rng = np.random.default_rng(2)
    info = np.iinfo(dt)
    a = rng.integers(info.min, info.max, size=50_000, dtype=dt, endpoint=True)
    inc = np.cumsum(a, dtype=dt)  # numpy wraps in the element type
    exc = np.concatenate([np.zeros(1, dt), inc[:-1]])
    assert (o.scan(a, True) == inc).all()
    assert (o.scan(a, False) == exc).all()
    assert (o.scan(a, True, nthreads=4) == inc).all()


@pytest.mark.parametrize("inclusive", [False, True])
def test_scan_mt_lookback_equals_sequential(inclusive):
    a = o.gen("u8_u32", 1_000_003, 3)
    assert (o.scan(a, inclusive, nthreads=6) == o.scan(a, inclusive)).all()


def test_scan_f64_against_numpy():
    a = o.gen("normal_f32", 100_000, 11)
    ref, ab = o.scan_f64(a, True)
    np.testing.assert_allclose(ref, np.cumsum(a.astype(np.float64)), rtol=0, atol=1e-9)
    np.testing.assert_allclose(ab, np.cumsum(np.abs(a.astype(np.float64))), rtol=1e-12)
    ex, _ = o.scan_f64(a, False)
    assert ex[0] == 0 and np.allclose(ex[1:], ref[:-1], atol=1e-9)


SCAN_OPS = {o.OP_SUM: np.add, o.OP_MIN: np.minimum, o.OP_MAX: np.maximum}


def np_scan_init(a, inclusive, npop, init):
    """numpy's in-order accumulate over [init] + a: exclusive = all but the
    last, inclusive = all but the first (np.add.accumulate wraps integers in
    the element type and adds floats left to right)."""
    acc = npop.accumulate(np.concatenate([np.array([init], a.dtype), a]), dtype=a.dtype)
    return acc[1:] if inclusive else acc[:-1]


@pytest.mark.parametrize("dt", [np.int32, np.uint32, np.float32, np.int64, np.uint64, np.float64])
@pytest.mark.parametrize("op", [o.OP_SUM, o.OP_MIN, o.OP_MAX])
@pytest.mark.parametrize("inclusive", [False, True])
def test_scan_op_init_vs_numpy_accumulate(dt, op, inclusive):
    # DeviceScan::ExclusiveScan / InclusiveScan (device_scan.h:114-178)
    rng = np.random.default_rng(op * 10 + inclusive)
    n = 30_001
    if np.dtype(dt).kind == "f":
        a = (rng.standard_normal(n) * 1000).astype(dt)
        init = dt(-123.25)
    else:
        info = np.iinfo(dt)
        a = rng.integers(info.min, info.max, n, dtype=dt, endpoint=True)
        init = dt(info.max // 3)
    got = o.scan_op(a, inclusive, op, init)
    ref = np_scan_init(a, inclusive, SCAN_OPS[op], init)
    assert got.tobytes() == ref.tobytes()


@pytest.mark.parametrize("inclusive", [False, True])
def test_scan_op_identity_init_is_the_sum_scan_and_constant_closed_form(inclusive):
    a = o.gen("reduce_i32", 10_007, 5)
    assert (o.scan_op(a, inclusive, o.OP_SUM) == o.scan(a, inclusive)).all()
    assert (o.scan_op(a, inclusive, o.OP_SUM, 0) == o.scan(a, inclusive)).all()
    # constant input c with init z: exclusive z + i c, inclusive z + (i + 1) c (int64, no wrap)
    c, z, n = np.int64(-7), np.int64(10**12), 5000
    i = np.arange(n, dtype=np.int64)
    got = o.scan_op(np.full(n, c), inclusive, o.OP_SUM, z)
    assert (got == z + (i + inclusive) * c).all()
    # Min from an init below every element stays at init; Max from lowest() is numpy's
    assert (o.scan_op(a, inclusive, o.OP_MIN, np.int32(-2**31)) == -2**31).all()
    assert (o.scan_op(a, True, o.OP_MAX) == np.maximum.accumulate(a)).all()


def test_scan_op_planted_mistakes_are_caught():
    """Plausible restatement mistakes, applied to the oracle's own output,
    fail the numpy check: init dropped, init folded in twice (as the
    reference's first tile does once per warp), exclusive / inclusive
    shifted by one, min for max."""
    a = o.gen("reduce_i32", 4096, 9).astype(np.int64)
    z = np.int64(1000)
    ref_ex = np_scan_init(a, False, np.add, z)
    ref_in = np_scan_init(a, True, np.add, z)
    assert (o.scan_op(a, False, o.OP_SUM, z) == ref_ex).all()
    planted = {
        "init dropped": o.scan_op(a, False, o.OP_SUM, z) - z,
        "init twice": o.scan_op(a, False, o.OP_SUM, z) + z,
        "inclusive for exclusive": o.scan_op(a, True, o.OP_SUM, z),
    }
    for what, bad in planted.items():
        assert not (bad == ref_ex).all(), what
    assert not (o.scan_op(a, True, o.OP_MIN, z) == np_scan_init(a, True, np.maximum, z)).all()
    assert not (o.scan_op(a, False, o.OP_SUM, z) == ref_in).all()


def test_lookback_kat_102400_tiles():
    # decoupled_look_back.cpp:57-174: aggregate 1 per tile -> exclusive i, inclusive i+1
    ex, inc = o.lookback_kat(102400, 8)
    assert (ex == np.arange(102400)).all() and (inc == np.arange(1, 102401)).all()


@pytest.mark.parametrize("nthreads", [1, 4, 8])
@pytest.mark.parametrize("width", [1, 16, 64])
def test_bounded_lookback_exact_when_every_tile_publishes(nthreads, width):
    # the bounded wait changes nothing while every predecessor publishes:
    # numpy's wrapping cumsum, status word 0
    agg = o.words(77, 20000).astype(np.uint32).view(np.int32)
    ex, inc, st = o.lookback_bounded(agg, nthreads, width=width)
    ref = np.cumsum(agg.astype(np.int64)).astype(np.int32)  # wraps like int32
    assert st == 0
    assert (inc == ref).all() and ex[0] == 0 and (ex[1:] == ref[:-1]).all()


@pytest.mark.parametrize("withhold", [0, 1, 7, 3000, 4095])
@pytest.mark.parametrize("nthreads", [1, 8])
def test_bounded_lookback_withheld_predecessor_reports_timeout(withhold, nthreads):
    """A tile that never publishes: every wait still ends, the status word
    carries LOOKBACK_TIMEOUT, and the library decodes that word to
    LCPP_ERR_LOOKBACK_TIMEOUT (-5), as lcpp_temp_status reports a device
    give-up.  Tiles before the withheld one are exact; tiles after it lost
    exactly its aggregate (an unpublished word reads as 0)."""
    import lc_parallel_primitive_amd as lcpp

    n = 4096
    agg = o.words(78, n).astype(np.uint32).view(np.int32)
    ex, inc, st = o.lookback_bounded(agg, nthreads, withhold=withhold, spin_limit=2000)
    ref = np.cumsum(agg.astype(np.int64))
    last = withhold == n - 1  # no tile waits on the last one
    assert (st & 1) == (0 if last else 1)
    assert lcpp.lib().lcpp_device_status_decode(st) == (0 if last else -5)
    w = withhold
    assert (inc[:w] == ref[:w].astype(np.int32)).all()
    lost = (ref[w + 1:] - int(agg[w])).astype(np.int32)
    assert (inc[w + 1:] == lost).all()



# ------------------------------------------------------------------ radix sort
@pytest.mark.parametrize("dt", SORT_DTYPES)
@pytest.mark.parametrize("nthreads", [1, 4])
def test_sort_keys_vs_numpy(dt, nthreads):
    rng = np.random.default_rng(3)
    n = 70_001
    if np.issubdtype(dt, np.floating):
        a = (rng.standard_normal(n) * 1e3).astype(dt)
        a[::97] = 0.0
        a[::89] = -0.0
    else:
        info = np.iinfo(dt)
        a = rng.integers(info.min, info.max, size=n, dtype=dt, endpoint=True)
    got = o.radix_sort(a, nthreads=nthreads, tile_items=1024)
    ref = np.sort(a, kind="stable")
    assert (got == ref).all()  # value equality (+0 == -0)
    # stability of +-0: the original order of zeros is kept
    if np.issubdtype(dt, np.floating):
        zeros_in = np.signbit(a[a == 0])
        zeros_out = np.signbit(got[got == 0])
        assert (zeros_in == zeros_out).all()


def test_sort_kat_reversed_keys():
    # device_radix_sort_one_sweep.cpp:120-151: keys N-1..0
    for k in (0, 1, 5, 12, 17):
        n = 1 << k
        a = np.arange(n - 1, -1, -1, dtype=np.uint32)
        assert (o.radix_sort(a, tile_items=512) == np.arange(n, dtype=np.uint32)).all()


@pytest.mark.parametrize("n", [32, 256, 4096])
def test_sort_kat_float_golden(n):
    # device_radix_sort_one_sweep.cpp:61-118 (ascending and descending)
    asc = golden(f"sort_float_{n}_asc_in_f32.bin", np.float32)
    desc = golden(f"sort_float_{n}_desc_in_f32.bin", np.float32)
    assert (o.radix_sort(asc) == golden(f"sort_float_{n}_asc_expect_f32.bin", np.float32)).all()
    assert (o.radix_sort(desc, descending=True) == golden(f"sort_float_{n}_desc_expect_f32.bin", np.float32)).all()


def test_sort_kat_pairs_golden():
    k = golden("sort_pairs_16384_keys_in_u32.bin", np.uint32)
    v = golden("sort_pairs_16384_vals_in_f32.bin", np.float32)
    ko, vo = o.radix_sort(k, v, nthreads=3, tile_items=1024)
    assert (ko == golden("sort_pairs_16384_keys_expect_u32.bin", np.uint32)).all()
    assert (vo == golden("sort_pairs_16384_vals_expect_f32.bin", np.float32)).all()


def stable_descending_perm(a: np.ndarray) -> np.ndarray:
    """Permutation that sorts `a` into non-increasing order, equal keys in
    input order (an independent construction: a stable ascending argsort of
    the reversed array, reversed back)."""
    n = a.size
    return (n - 1 - np.argsort(a[::-1], kind="stable"))[::-1]


@pytest.mark.parametrize("dt", SORT_DTYPES)
def test_sort_keys_descending_vs_numpy(dt):
    rng = np.random.default_rng(11)
    n = 50_003
    if np.issubdtype(dt, np.floating):
        a = (rng.standard_normal(n) * 1e3).astype(dt)
        a[::97] = 0.0
        a[::89] = -0.0
    else:
        info = np.iinfo(dt)
        a = rng.integers(info.min, info.max, size=n, dtype=dt, endpoint=True)
        a[::50] = a[7]  # duplicates
    got = o.radix_sort(a, descending=True, nthreads=3, tile_items=1024)
    ref = a[stable_descending_perm(a)]
    assert (got == ref).all()
    if np.issubdtype(dt, np.floating):  # +-0 compare equal and keep input order
        assert (np.signbit(a[a == 0]) == np.signbit(got[got == 0])).all()


def float_total_order_perm(a: np.ndarray, descending: bool = False) -> np.ndarray:
    """Permutation that orders float keys as an IEEE-754 radix sort does, built
    from value comparisons and NaN signs and bit patterns only (not from the
    key twiddle): negative NaNs (larger bit patterns first), then every other
    value in numeric order with -0.0 == +0.0, then positive NaNs (smaller bit
    patterns first); equal keys in input order.  Descending reverses the
    order of distinct keys and keeps equal keys in input order."""
    bits = a.view(np.uint32 if a.dtype.itemsize == 4 else np.uint64)
    idx = np.arange(a.size)
    nan = np.isnan(a)
    neg = np.signbit(a)
    negnan, posnan, num = idx[nan & neg], idx[nan & ~neg], idx[~nan]
    up = lambda ix, key: ix[np.argsort(key[ix], kind="stable")]
    down = lambda ix, key: ix[stable_descending_perm(key[ix])]
    if descending:
        return np.concatenate([down(posnan, bits), down(num, a), up(negnan, bits)])
    return np.concatenate([down(negnan, bits), up(num, a), up(posnan, bits)])


def test_float_total_order_perm_small_case():
    f = np.float32
    nan = lambda b: np.array([b], np.uint32).view(f)[0]
    a = np.array([1.0, nan(0x7FC00001), -0.0, -np.inf, nan(0xFFC00000), 0.0, np.inf, nan(0x7FC00000),
                  nan(0xFFC00001), -2.5, 1.0], f)
    assert float_total_order_perm(a).tolist() == [8, 4, 3, 9, 2, 5, 0, 10, 6, 7, 1]
    assert float_total_order_perm(a, descending=True).tolist() == [1, 7, 6, 0, 10, 2, 5, 9, 3, 4, 8]


@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("descending", [False, True])
def test_sort_special_floats_vs_total_order(dt, descending):
    from conftest import special_float_keys

    a = special_float_keys(dt, 60_001, seed=21)
    perm = float_total_order_perm(a, descending)
    v = np.arange(a.size, dtype=np.uint32)
    ko = o.radix_sort(a, descending=descending, nthreads=3, tile_items=1024)
    ko2, vo = o.radix_sort(a, v, descending=descending, nthreads=3, tile_items=1024)
    assert ko.tobytes() == a[perm].tobytes()  # bit-exact: NaN payloads, -0.0 / +0.0 order
    assert ko2.tobytes() == a[perm].tobytes() and (vo == perm).all()


def test_stable_descending_perm_is_independent_of_the_oracle():
    a = np.array([3, 1, 3, 2, 1, 3], dtype=np.uint32)
    assert stable_descending_perm(a).tolist() == [0, 2, 5, 3, 1, 4]


def test_sort_pairs_descending_stability():
    k = o.gen("keys_u64_low16", 200_000, 8)
    v = np.arange(k.size, dtype=np.uint32)
    ko, vo = o.radix_sort(k, v, descending=True, nthreads=4, tile_items=2048)
    perm = stable_descending_perm(k)
    assert (vo == perm).all() and (ko == k[perm]).all()


def test_sort_kat_pairs_descending_golden():
    # device_radix_sort_one_sweep.cpp:153-279, SortPairsDescending leg
    k = golden("sort_pairs_desc_16384_keys_in_u32.bin", np.uint32)
    v = golden("sort_pairs_desc_16384_vals_in_f32.bin", np.float32)
    ko, vo = o.radix_sort(k, v, descending=True, nthreads=2, tile_items=1024)
    assert (ko == golden("sort_pairs_desc_16384_keys_expect_u32.bin", np.uint32)).all()
    assert (vo == golden("sort_pairs_desc_16384_vals_expect_f32.bin", np.float32)).all()


def test_sort_pairs_stability_vs_numpy_argsort():
    k = o.gen("keys_u64_low16", 300_000, 4)
    v = np.arange(k.size, dtype=np.uint32)
    ko, vo = o.radix_sort(k, v, nthreads=4, tile_items=2048)
    perm = np.argsort(k, kind="stable")
    assert (vo == perm).all() and (ko == k[perm]).all()
    assert o.check_stable_pairs_u64_u32(k, ko, vo)


def test_stability_checker_catches_planted_mistakes():
    k = o.gen("keys_u64_low16", 50_000, 5) & np.uint64(0xFF)  # many duplicates
    v = np.arange(k.size, dtype=np.uint32)
    ko, vo = o.radix_sort(k, v)
    assert o.check_stable_pairs_u64_u32(k, ko, vo)
    # swap two equal keys' values -> unstable
    i = int(np.nonzero(ko[1:] == ko[:-1])[0][0])
    vo2 = vo.copy(); vo2[[i, i + 1]] = vo2[[i + 1, i]]
    assert not o.check_stable_pairs_u64_u32(k, ko, vo2)
    # duplicate a value -> not a permutation
    vo3 = vo.copy(); vo3[5] = vo3[6]
    assert not o.check_stable_pairs_u64_u32(k, ko, vo3)
    # break key order
    ko4 = ko.copy(); ko4[[0, -1]] = ko4[[-1, 0]]
    assert not o.check_stable_pairs_u64_u32(k, ko4, vo)


def test_sorted_permutation_checker():
    a = o.gen("keys_u32", 100_000, 6)
    s = np.sort(a)
    assert o.check_sorted_permutation_u32(a, s)
    s2 = s.copy(); s2[100] = s2[101]  # keeps order, changes multiset (if distinct)
    if s[100] != s[101]:
        assert not o.check_sorted_permutation_u32(a, s2)
    s3 = s.copy(); s3[[10, 20]] = s3[[20, 10]]
    assert not o.check_sorted_permutation_u32(a, s3) or s[10] == s[20]


def test_sort_lsd_mistake_is_caught():
    """A planted mistake in a sort (one 8-bit digit pass skipped) must be
    visible to the same comparison the GPU parity tests use."""
    a = o.gen("keys_u32", 10_000, 7)
    bad = a[np.argsort(a & np.uint32(0xFFFF00FF), kind="stable")]
    assert not (bad == o.radix_sort(a)).all()


# ------------------------------------------------------------------ segment reduce
def test_segment_reduce_kat_golden():
    # device_segment_reduce.cpp:62-125
    a = golden("segment_shuffled_1024_i32.bin", np.int32)
    b = golden("segment_shuffled_1024_begin_u32.bin", np.uint32)
    e = golden("segment_shuffled_1024_end_u32.bin", np.uint32)
    exp = golden("segment_shuffled_1024_expect_i32.bin", np.int32)
    assert (o.segment_reduce(o.OP_SUM, a, b, e) == exp).all()


def test_segment_reduce_vs_numpy():
    b, e = o.segments(1, 2, 200_000, 1500)
    a = o.gen("reduce_i32", 200_000, 3)
    ref = np.array([a[x:y].astype(np.int64).sum() for x, y in zip(b, e)]).astype(np.int32)
    assert (o.segment_reduce(o.OP_SUM, a, b, e) == ref).all()
    assert (o.segment_reduce_mt(a, b, e, 4) == ref).all()
    f = o.gen("normal_f32", 200_000, 3)
    s, ab = o.segment_reduce_f64(f, b, e)
    ref64 = np.array([f[x:y].astype(np.float64).sum() for x, y in zip(b, e)])
    np.testing.assert_allclose(s, ref64, rtol=0, atol=1e-9)
    assert (s[b == e] == 0).all()


def test_segment_reduce_empty_and_inverted_segments():
    a = np.arange(10, dtype=np.int32)
    b = np.array([0, 3, 3, 7, 9], np.uint32)
    e = np.array([3, 3, 1, 10, 9], np.uint32)  # [0,3), empty, inverted (empty), [7,10), empty
    assert list(o.segment_reduce(o.OP_SUM, a, b, e)) == [3, 0, 0, 24, 0]


# ------------------------------------------------------------------ scan by key / reduce by key
BYKEY_VALUE_DTYPES = [np.int32, np.uint32, np.int64, np.uint64]


def run_keys(n: int, mean_len: float, seed: int, dtype=np.int32) -> np.ndarray:
    """Keys made of runs with geometric lengths (consecutive runs differ)."""
    rng = np.random.default_rng(seed)
    heads = rng.random(n) < 1.0 / mean_len
    heads[0] = True
    return (np.cumsum(heads) * 7 % 1000).astype(dtype)


def heads_of(keys: np.ndarray) -> np.ndarray:
    h = np.ones(keys.size, bool)
    h[1:] = keys[1:] != keys[:-1]
    return h


def np_scan_by_key_sum(keys, v, inclusive, init):
    """Segmented sums as differences of one global cumsum (wraparound in the
    element type): independent of the oracle's per-element restart."""
    with np.errstate(over="ignore"):
        c = np.cumsum(v, dtype=v.dtype)
        start = np.maximum.accumulate(np.where(heads_of(keys), np.arange(v.size), 0))
        base = np.where(start > 0, c[np.maximum(start - 1, 0)], v.dtype.type(0)).astype(v.dtype)
        incl = (c - base).astype(v.dtype)
        out = incl if inclusive else (incl - v).astype(v.dtype)
        return (out + v.dtype.type(init)).astype(v.dtype)


def test_scan_by_key_kat_exclusive_ones():
    # device_scan_test.cpp:111-167: keys i/100, values 1 -> i % 100
    for k in range(5, 17):
        n = 1 << k
        keys = (np.arange(n) // 100).astype(np.int32)
        got = o.scan_by_key(keys, np.ones(n, np.int32), inclusive=False)
        assert (got == np.arange(n) % 100).all()


@pytest.mark.parametrize("dt", BYKEY_VALUE_DTYPES)
@pytest.mark.parametrize("inclusive", [False, True])
def test_scan_by_key_sum_vs_numpy_cumsum_differences(dt, inclusive):
    n = 50_000
    keys = run_keys(n, 37, 5)
    info = np.iinfo(dt)
    v = np.random.default_rng(6).integers(info.min, info.max, n, dtype=dt, endpoint=True)
    for init in (0, 12345):
        got = o.scan_by_key(keys, v, inclusive, o.OP_SUM, init)
        assert (got == np_scan_by_key_sum(keys, v, inclusive, init)).all()


@pytest.mark.parametrize("op", [o.OP_MIN, o.OP_MAX])
@pytest.mark.parametrize("inclusive", [False, True])
def test_scan_by_key_min_max_vs_numpy_accumulate(op, inclusive):
    n = 20_000
    keys = run_keys(n, 25, 7, np.uint32)
    v = np.random.default_rng(8).integers(-10**6, 10**6, n).astype(np.int32)
    init = np.int32(500_000 if op == o.OP_MIN else -500_000)
    npop = np.minimum if op == o.OP_MIN else np.maximum
    ref = np.empty_like(v)
    h = np.flatnonzero(heads_of(keys))
    for s, e in zip(h, list(h[1:]) + [n]):
        acc = npop.accumulate(v[s:e])
        if inclusive:
            ref[s:e] = npop(acc, init)
        else:
            ref[s] = init
            ref[s + 1:e] = npop(acc[:-1], init)
    assert (o.scan_by_key(keys, v, inclusive, op, init) == ref).all()


def test_scan_by_key_special_cases():
    v = o.gen("reduce_i32", 4097, 11)
    one_run = np.full(v.size, 9, np.int64)
    for inclusive in (False, True):
        assert (o.scan_by_key(one_run, v, inclusive) == o.scan(v, inclusive)).all()
    distinct = np.arange(v.size, dtype=np.uint64)
    assert (o.scan_by_key(distinct, v, False, o.OP_SUM, 3) == 3).all()
    assert (o.scan_by_key(distinct, v, True, o.OP_SUM, 3) == v + 3).all()
    assert (o.scan_by_key(distinct, v, True, o.OP_MAX, 0) == np.maximum(v, 0)).all()
    assert o.scan_by_key(np.empty(0, np.int32), np.empty(0, np.int32), True).size == 0


def test_scan_by_key_float_key_equality():
    # keys compared as floats: -0.0 == +0.0 (one run), NaN != NaN (each its own run)
    keys = np.array([1.0, -0.0, 0.0, np.nan, np.nan, 2.0], np.float32)
    v = np.ones(6, np.int32)
    assert list(o.scan_by_key(keys, v, True)) == [1, 1, 2, 1, 1, 1]
    uk, ag = o.reduce_by_key(keys, v)
    assert list(ag) == [1, 2, 1, 1, 1] and uk.size == 5


def test_scan_by_key_f64_and_float_values():
    n = 30_000
    keys = run_keys(n, 50, 12, np.float64)
    f = o.gen("normal_f32", n, 13)
    for inclusive in (False, True):
        s, ab = o.scan_by_key_f64(keys, f, inclusive)
        ref = np_scan_by_key_sum(keys, f.astype(np.float64), inclusive, 0)
        np.testing.assert_allclose(s, ref, rtol=0, atol=1e-9)
        got = o.scan_by_key(keys, f, inclusive).astype(np.float64)
        assert (np.abs(got - s) <= 1e-5 * ab + 1e-30).all()


def test_scan_by_key_planted_missing_head_is_caught():
    keys = run_keys(5000, 20, 14)
    v = np.ones(5000, np.int32)
    good = o.scan_by_key(keys, v, True)
    bad_keys = keys.copy()
    h = np.flatnonzero(heads_of(keys))
    bad_keys[h[10]] = bad_keys[h[10] - 1]  # merge two runs at one position
    assert not (np_scan_by_key_sum(bad_keys, v, True, 0) == good).all()


def test_reduce_by_key_kat_shuffled_chunks():
    # device_reduce_test.cpp:229-289: keys i/100 over the shuffled 0..4095
    a = golden("reduce_shuffled_4096_i32.bin", np.int32)
    keys = (np.arange(a.size) // 100).astype(np.int32)
    uk, ag = o.reduce_by_key(keys, a)
    assert uk.size == 41 and (uk == np.arange(41)).all()
    assert (ag == np.array([a[i * 100:(i + 1) * 100].sum() for i in range(41)])).all()


@pytest.mark.parametrize("dt", BYKEY_VALUE_DTYPES + [np.float32, np.float64])
@pytest.mark.parametrize("op", [o.OP_SUM, o.OP_MIN, o.OP_MAX])
def test_reduce_by_key_vs_numpy_reduceat(dt, op):
    n = 40_000
    keys = run_keys(n, 9, 15, np.int64)
    dt = np.dtype(dt)
    if dt.kind == "f":
        v = np.random.default_rng(16).integers(-1000, 1000, n).astype(dt)  # exact in any order
    else:
        info = np.iinfo(dt)
        v = np.random.default_rng(16).integers(info.min, info.max, n, dtype=dt, endpoint=True)
    h = np.flatnonzero(heads_of(keys))
    npop = {o.OP_SUM: np.add, o.OP_MIN: np.minimum, o.OP_MAX: np.maximum}[op]
    with np.errstate(over="ignore"):
        ref = npop.reduceat(v, h).astype(dt)
    uk, ag = o.reduce_by_key(keys, v, op)
    assert uk.size == h.size == 1 + np.count_nonzero(np.diff(keys))
    assert (uk == keys[h]).all() and (ag == ref).all()


def test_reduce_by_key_f64_and_edges():
    n = 20_000
    keys = run_keys(n, 3, 17, np.uint32)
    f = o.gen("normal_f32", n, 18)
    s, ab = o.reduce_by_key_f64(keys, f)
    h = np.flatnonzero(heads_of(keys))
    np.testing.assert_allclose(s, np.add.reduceat(f.astype(np.float64), h), rtol=0, atol=1e-9)
    assert (ab >= np.abs(s)).all()
    uk, ag = o.reduce_by_key(np.empty(0, np.int32), np.empty(0, np.int32))
    assert uk.size == 0 and ag.size == 0
    uk, ag = o.reduce_by_key(np.array([5], np.int32), np.array([-7], np.int32))
    assert list(uk) == [5] and list(ag) == [-7]


# ------------------------------------------------------------------ segment Min/Max/Arg*, fixed-size
SHUFFLED_1024 = "segment_shuffled_1024_i32.bin"


def test_segment_kat_fixed_sum_closed_form():
    # device_segment_reduce.cpp fixed_segment_reduce: 0..1023 in segments of 32
    a = np.arange(1024, dtype=np.int32)
    b, e = o.fixed_segments(32, 32)
    assert (o.segment_reduce(o.OP_SUM, a, b, e) == np.array([32 * 32 * i + 496 for i in range(32)])).all()


def test_segment_kat_argmax_shuffled():
    # device_segment_reduce.cpp segment_reduce_arg_max: shuffled 0..1023, 11 segments of <= 100
    a = golden(SHUFFLED_1024, np.int32)
    b = np.arange(0, 1024, 100, dtype=np.uint32)
    e = np.minimum(b + 100, 1024).astype(np.uint32)
    v, i = o.segment_reduce_arg(True, a, b, e)
    assert b.size == 11
    assert (v == np.array([a[x:y].max() for x, y in zip(b, e)])).all()
    assert (i == np.array([a[x:y].argmax() for x, y in zip(b, e)])).all()


def test_segment_kat_fixed_argmin_shuffled():
    # device_segment_reduce.cpp fixed_segment_reduce_arg_min: shuffled 0..1023, fixed 32
    a = golden(SHUFFLED_1024, np.int32)
    b, e = o.fixed_segments(32, 32)
    v, i = o.segment_reduce_arg(False, a, b, e)
    assert (v == a.reshape(32, 32).min(axis=1)).all() and (i == a.reshape(32, 32).argmin(axis=1)).all()


@pytest.mark.parametrize("dt", [np.int32, np.uint32, np.float32, np.int64, np.uint64, np.float64])
def test_segment_min_max_init_vs_numpy(dt):
    b, e = o.segments(11, 12, 50_000, 700)
    e[::9] = b[::9]  # extra empty segments
    dt = np.dtype(dt)
    rng = np.random.default_rng(13)
    a = (rng.standard_normal(50_000) * 1000).astype(dt) if dt.kind == "f" else \
        rng.integers(np.iinfo(dt).min, np.iinfo(dt).max, 50_000, dtype=dt, endpoint=True)
    for op, npop, ident in ((o.OP_MIN, np.min, np.inf), (o.OP_MAX, np.max, -np.inf)):
        base = dt.type(a[100])
        got = o.segment_reduce(op, a, b, e, init=base)
        ref = np.array([npop(np.append(a[x:y], base)) for x, y in zip(b, e)], dt)
        assert (got == ref).all()
        got0 = o.segment_reduce(op, a, b, e)
        lim = (np.finfo(dt) if dt.kind == "f" else np.iinfo(dt))
        empty_val = lim.max if op == o.OP_MIN else (lim.min if dt.kind != "f" else -lim.max)
        assert all(g == (npop(a[x:y]) if y > x else empty_val) for g, x, y in zip(got0, b, e))


def test_segment_sum_init_wraps():
    a = np.array([2**31 - 1, 5], np.int32)
    b, e = np.array([0, 0], np.uint32), np.array([2, 0], np.uint32)
    assert list(o.segment_reduce(o.OP_SUM, a, b, e, init=np.int32(10))) == [np.int32(-2**31 + 14), 10]


@pytest.mark.parametrize("dt", [np.int32, np.float32, np.uint64, np.float64])
def test_segment_arg_vs_numpy(dt):
    b, e = o.segments(14, 15, 40_000, 500)
    e[::13] = b[::13]
    dt = np.dtype(dt)
    rng = np.random.default_rng(16)
    a = rng.integers(0, 40, 40_000).astype(dt)  # many ties
    vmin, imin = o.segment_reduce_arg(False, a, b, e)
    vmax, imax = o.segment_reduce_arg(True, a, b, e)
    lim = np.finfo(dt) if dt.kind == "f" else np.iinfo(dt)
    for s, (x, y) in enumerate(zip(b, e)):
        seg = a[x:y]
        if y <= x:
            assert imin[s] == 1 and imax[s] == 1 and vmin[s] == lim.max
            assert vmax[s] == (lim.min if dt.kind != "f" else -lim.max)
            continue
        assert imin[s] == seg.argmin() and vmin[s] == seg.min()  # ties: smallest index
        assert imax[s] == seg.size - 1 - seg[::-1].argmax() and vmax[s] == seg.max()  # ties: largest index


def test_segment_arg_infinite_values():
    a = np.array([-np.inf, -np.inf, np.inf, np.inf], np.float32)
    b, e = np.array([0, 2], np.uint32), np.array([2, 4], np.uint32)
    v, i = o.segment_reduce_arg(True, a, b, e)
    assert list(i) == [1, 1] and v[0] == -np.inf and v[1] == np.inf
    v, i = o.segment_reduce_arg(False, a, b, e)
    assert list(i) == [0, 0]
