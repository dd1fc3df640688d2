"""DeviceRadixSort::SortKeys/SortPairs(Descending) (onesweep) on the GPU through the C ABI.
Bit-exact against the oracle (itself pinned against numpy stable sorts and
the reference's known answers); pairs are checked for stability; full-size
configurations use O(N) sortedness + multiset / stability checkers."""
import numpy as np
import pytest

from conftest import golden, log
from oracle import oracle as o

pytestmark = pytest.mark.gpu

KEY_DTYPES = [np.uint32, np.int32, np.float32, np.uint64, np.int64, np.float64]
SIZES = [1, 2, 63, 64, 65, 4095, 4096, 4097, 8191, 100_003]


def sort_keys(d_in, n, dtype, pad=0, descending=False):
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceRadixSort

    out = g.empty(n, dtype, pad=pad)
    tmp = g.temp(DeviceRadixSort.GetSortKeysTempStorageBytes(np.dtype(dtype).name, n))
    s = DeviceRadixSort()
    (s.SortKeysDescending if descending else s.SortKeys)(tmp, d_in, out, n)
    return out


def sort_pairs(dk, dv, n, kdt, vdt, descending=False):
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceRadixSort

    ko = g.empty(n, kdt)
    vo = g.empty(n, vdt)
    tmp = g.temp(DeviceRadixSort.GetSortPairsTempStorageBytes(np.dtype(kdt).name, np.dtype(vdt).name, n))
    s = DeviceRadixSort()
    (s.SortPairsDescending if descending else s.SortPairs)(tmp, dk, ko, dv, vo, n)
    return ko, vo


def same_bits(a, b):
    return a.tobytes() == b.tobytes()


def test_kat_reversed_keys(gpu):
    # device_radix_sort_one_sweep.cpp:120-151: keys N-1..0, N = 2^0..2^23
    import gpu_util as g

    for k in range(24):
        n = 1 << k
        log(f"sort reversed n={n}")
        a = np.arange(n - 1, -1, -1, dtype=np.uint32)
        got = g.to_host(sort_keys(g.to_dev(a), n, np.uint32))
        assert (got == np.arange(n, dtype=np.uint32)).all()


@pytest.mark.parametrize("n", [32, 256, 4096])
def test_kat_float_keys_golden(gpu, n):
    # device_radix_sort_one_sweep.cpp:61-118 (SortKeys and SortKeysDescending)
    import gpu_util as g

    a = golden(f"sort_float_{n}_asc_in_f32.bin", np.float32)
    got = g.to_host(sort_keys(g.to_dev(a), n, np.float32))
    assert same_bits(got, golden(f"sort_float_{n}_asc_expect_f32.bin", np.float32))
    a = golden(f"sort_float_{n}_desc_in_f32.bin", np.float32)
    got = g.to_host(sort_keys(g.to_dev(a), n, np.float32, descending=True))
    assert same_bits(got, golden(f"sort_float_{n}_desc_expect_f32.bin", np.float32))


def test_kat_pairs_descending_golden(gpu):
    # device_radix_sort_one_sweep.cpp:153-279, SortPairsDescending leg
    import gpu_util as g

    k = golden("sort_pairs_desc_16384_keys_in_u32.bin", np.uint32)
    v = golden("sort_pairs_desc_16384_vals_in_f32.bin", np.float32)
    ko, vo = sort_pairs(g.to_dev(k), g.to_dev(v), k.size, np.uint32, np.float32, descending=True)
    assert same_bits(g.to_host(ko), golden("sort_pairs_desc_16384_keys_expect_u32.bin", np.uint32))
    assert same_bits(g.to_host(vo), golden("sort_pairs_desc_16384_vals_expect_f32.bin", np.float32))


def test_kat_pairs_golden(gpu):
    # device_radix_sort_one_sweep.cpp:153-279 procedure (uint keys, float values)
    import gpu_util as g

    k = golden("sort_pairs_16384_keys_in_u32.bin", np.uint32)
    v = golden("sort_pairs_16384_vals_in_f32.bin", np.float32)
    ko, vo = sort_pairs(g.to_dev(k), g.to_dev(v), k.size, np.uint32, np.float32)
    assert same_bits(g.to_host(ko), golden("sort_pairs_16384_keys_expect_u32.bin", np.uint32))
    assert same_bits(g.to_host(vo), golden("sort_pairs_16384_vals_expect_f32.bin", np.float32))


@pytest.mark.parametrize("dtype", KEY_DTYPES)
@pytest.mark.parametrize("n", SIZES)
def test_keys_vs_oracle(gpu, dtype, n):
    import gpu_util as g

    a = g.random_array(dtype, n, seed=n)
    log(f"sort keys {np.dtype(dtype).name} n={n}")
    d = g.to_dev(a)
    got = g.to_host(sort_keys(d, n, dtype))
    assert same_bits(got, o.radix_sort(a))  # bit-exact, including the order of -0.0 / +0.0
    assert same_bits(g.to_host(d), a)  # input preserved


@pytest.mark.parametrize("kdt,vdt", [(np.uint32, np.uint32), (np.uint64, np.uint32), (np.int32, np.float64),
                                     (np.float64, np.int64), (np.float32, np.uint32)])
@pytest.mark.parametrize("n", [1, 4097, 100_003])
def test_pairs_stable_vs_oracle(gpu, kdt, vdt, n):
    import gpu_util as g

    k = g.random_array(kdt, n, seed=3)
    if np.dtype(kdt).kind in "iu":
        k = k & np.array(0xFF, dtype=kdt)  # heavy duplication: stability matters
    v = np.arange(n, dtype=vdt)
    log(f"sort pairs {np.dtype(kdt).name}/{np.dtype(vdt).name} n={n}")
    ko, vo = sort_pairs(g.to_dev(k), g.to_dev(v), n, kdt, vdt)
    rk, rv = o.radix_sort(k, v)
    assert same_bits(g.to_host(ko), rk) and same_bits(g.to_host(vo), rv)


# Tiles hold 16384 keys (8192 when keys or values are 8 bytes) and the look-back
# groups them in batches of 8: sizes around 1, 2, 3, 5, 8, 9 and 25 batches,
# ragged and exact (a walk reads up to 8 batch words per poll in the kernels
# at four waves per SIMD, so the walks from batch 8 on take the unguarded
# window).
@pytest.mark.parametrize("kdt,vdt", [(np.uint32, None), (np.uint64, None), (np.uint32, np.uint32),
                                     (np.uint64, np.uint32)])
@pytest.mark.parametrize("tiles,delta", [(7, 0), (8, -1), (8, 0), (8, 1), (9, 0), (16, 0), (17, 5),
                                         (24, -3), (40, 7), (64, 0), (65, -1), (72, 3), (200, 11)])
def test_lookback_batch_boundaries(gpu, kdt, vdt, tiles, delta):
    import gpu_util as g

    tile = 8192 if np.dtype(kdt).itemsize == 8 or vdt is not None else 16384
    n = tiles * tile + delta
    k = g.random_array(kdt, n, seed=tiles * 7 + delta)
    log(f"sort batch boundaries {np.dtype(kdt).name}/{vdt and np.dtype(vdt).name} n={n}")
    if vdt is None:
        got = g.to_host(sort_keys(g.to_dev(k), n, kdt))
        assert same_bits(got, o.radix_sort(k))
    else:
        k = k & np.array(0xFFF, dtype=kdt)  # duplicates: stability across tiles and batches
        v = np.arange(n, dtype=vdt)
        ko, vo = sort_pairs(g.to_dev(k), g.to_dev(v), n, kdt, vdt)
        rk, rv = o.radix_sort(k, v)
        assert same_bits(g.to_host(ko), rk) and same_bits(g.to_host(vo), rv)


@pytest.mark.parametrize("dtype", KEY_DTYPES)
@pytest.mark.parametrize("n", [1, 65, 4097, 16385, 100_003])
def test_keys_descending_vs_oracle(gpu, dtype, n):
    import gpu_util as g

    a = g.random_array(dtype, n, seed=n + 1)
    log(f"sort keys descending {np.dtype(dtype).name} n={n}")
    d = g.to_dev(a)
    got = g.to_host(sort_keys(d, n, dtype, descending=True))
    assert same_bits(got, o.radix_sort(a, descending=True))
    assert same_bits(g.to_host(d), a)


@pytest.mark.parametrize("kdt,vdt", [(np.uint32, np.uint32), (np.uint64, np.uint32), (np.float32, np.uint32),
                                     (np.int64, np.float64)])
@pytest.mark.parametrize("n", [4097, 100_003])
def test_pairs_descending_stable_vs_oracle(gpu, kdt, vdt, n):
    import gpu_util as g

    k = g.random_array(kdt, n, seed=5)
    if np.dtype(kdt).kind in "iu":
        k = k & np.array(0xFF, dtype=kdt)
    v = np.arange(n, dtype=vdt)
    log(f"sort pairs descending {np.dtype(kdt).name}/{np.dtype(vdt).name} n={n}")
    ko, vo = sort_pairs(g.to_dev(k), g.to_dev(v), n, kdt, vdt, descending=True)
    rk, rv = o.radix_sort(k, v, descending=True)
    assert same_bits(g.to_host(ko), rk) and same_bits(g.to_host(vo), rv)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("descending", [False, True])
@pytest.mark.parametrize("n", [4097, 100_003])
def test_special_float_keys_vs_oracle(gpu, dtype, descending, n):
    # NaNs of both signs and several payloads, +-inf, subnormals, +-0: the
    # order is fixed by bit patterns (the oracle is pinned against an IEEE
    # total order built without the key twiddle)
    import gpu_util as g
    from conftest import special_float_keys

    a = special_float_keys(dtype, n, seed=n + 7)
    v = np.arange(n, dtype=np.uint32)
    log(f"sort special floats {np.dtype(dtype).name} n={n} descending={descending}")
    got = g.to_host(sort_keys(g.to_dev(a), n, dtype, descending=descending))
    assert same_bits(got, o.radix_sort(a, descending=descending))
    ko, vo = sort_pairs(g.to_dev(a), g.to_dev(v), n, dtype, np.uint32, descending=descending)
    rk, rv = o.radix_sort(a, v, descending=descending)
    assert same_bits(g.to_host(ko), rk) and same_bits(g.to_host(vo), rv)


def test_low_entropy_keys(gpu):
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 3_000_017
    d = datagen.keys_u32_and3(n)
    got = g.to_host(sort_keys(d, n, np.uint32))
    h = g.to_host(d)
    assert same_bits(got, o.radix_sort(h, nthreads=8))
    assert (h[:1000] == o.gen("keys_u32_and3", 1000, *datagen.SEED_SORT_AND3)).all()


@pytest.mark.parametrize("which", ["uniform", "and3"])
def test_full_size_u32(gpu, which):
    # BASELINE config C3a/C3b: 2^28 uint32 keys
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 1 << 28
    log(f"sort keys u32 full 2^28 {which}")
    d = datagen.keys_u32(n) if which == "uniform" else datagen.keys_u32_and3(n)
    got = g.to_host(sort_keys(d, n, np.uint32))
    h = g.to_host(d)
    assert o.check_sorted_permutation_u32(h, got)


def test_full_size_pairs_u64_index(gpu):
    # 2^27 uint64 keys with 16 random low bits, values = index
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 1 << 27
    log("sort pairs u64/u32 full 2^27")
    k = datagen.keys_u64_low16(n)
    v = datagen.iota_u32(n)
    ko, vo = sort_pairs(k, v, n, np.uint64, np.uint32)
    assert o.check_stable_pairs_u64_u32(g.to_host(k), g.to_host(ko), g.to_host(vo))


def test_full_size_pairs_u64_full_range_8_passes(gpu):
    # C4's shape with keys over the full 64-bit range: no digit pass is
    # trivial, so all 8 onesweep passes move keys and values
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 1 << 27
    log("sort pairs u64 (full range)/u32 2^27, 8 passes")
    k = datagen.keys_u64(n)
    v = datagen.iota_u32(n)
    ko, vo = sort_pairs(k, v, n, np.uint64, np.uint32)
    assert o.check_stable_pairs_u64_u32(g.to_host(k), g.to_host(ko), g.to_host(vo))


def test_full_size_u32_descending(gpu):
    # C3a input sorted with SortKeysDescending: the reversed output must be an
    # ascending permutation of the input
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 1 << 28
    log("sort keys u32 descending full 2^28")
    d = datagen.keys_u32(n)
    got = g.to_host(sort_keys(d, n, np.uint32, descending=True))
    assert o.check_sorted_permutation_u32(g.to_host(d), np.ascontiguousarray(got[::-1]))


def test_full_size_pairs_u64_descending(gpu):
    # C4 input with SortPairsDescending: a stable descending sort of k is a
    # stable ascending sort of ~k, which the O(N) stability checker verifies
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 1 << 27
    log("sort pairs u64/u32 descending full 2^27")
    k = datagen.keys_u64_low16(n)
    v = datagen.iota_u32(n)
    ko, vo = sort_pairs(k, v, n, np.uint64, np.uint32, descending=True)
    hk = g.to_host(k)
    assert o.check_stable_pairs_u64_u32(~hk, ~g.to_host(ko), g.to_host(vo))


@pytest.mark.parametrize("n", [1, 4097, 100_003, 1 << 20])
@pytest.mark.parametrize("kdt", [np.uint32, np.int64])
@pytest.mark.parametrize("descending", [False, True])
def test_skewed_digits_stable(gpu, n, kdt, descending):
    """Keys where one digit value dominates every pass (the hot-digit ranking
    path): 90 % one key, the rest random; values = index check stability."""
    import gpu_util as g

    rng = np.random.default_rng(n)
    info = np.iinfo(kdt)
    k = np.full(n, kdt(0x5A5A5A5A) if info.bits == 32 else kdt(0x1234567890), dtype=kdt)
    mask = rng.random(n) < 0.1
    k[mask] = rng.integers(info.min, info.max, mask.sum(), dtype=kdt, endpoint=True)
    v = np.arange(n, dtype=np.uint32)
    log(f"skewed pairs n={n} {np.dtype(kdt).name} desc={descending}")
    ko, vo = sort_pairs(g.to_dev(k), g.to_dev(v), n, kdt, np.uint32, descending=descending)
    ek, ev = o.radix_sort(k, v, descending=descending)
    assert same_bits(g.to_host(ko), ek) and same_bits(g.to_host(vo), ev)


def test_constant_keys_all_lanes_hot(gpu):
    import gpu_util as g

    n = (1 << 20) + 77
    k = np.full(n, 7, np.uint32)
    v = np.arange(n, dtype=np.uint32)
    ko, vo = sort_pairs(g.to_dev(k), g.to_dev(v), n, np.uint32, np.uint32)
    assert (g.to_host(ko) == 7).all() and (g.to_host(vo) == v).all()


# Digit passes in which every key has the same digit are skipped; these masks
# leave trivial passes at the start, in the middle and at the end, and one
# pass or several that move data (the pass plan's buffer ping-pong).
@pytest.mark.parametrize("kdt,mask", [(np.uint32, 0x0000FF00), (np.uint32, 0xFF00FF00), (np.uint32, 0x00FF0000),
                                      (np.uint32, 0xFF000000), (np.uint32, 0x00FFFF00), (np.uint64, 0x00FF00FF00FF00FF),
                                      (np.uint64, 0xFF00000000000000), (np.uint64, 0x0000FFFF00000000)])
@pytest.mark.parametrize("descending", [False, True])
def test_trivial_passes_skipped(gpu, kdt, mask, descending):
    import gpu_util as g

    n = 300_007
    k = g.random_array(kdt, n, seed=11) & np.array(mask, dtype=kdt)
    v = np.arange(n, dtype=np.uint32)
    log(f"sort trivial passes {np.dtype(kdt).name} mask={mask:#x} descending={descending}")
    got = g.to_host(sort_keys(g.to_dev(k), n, kdt, descending=descending))
    assert same_bits(got, o.radix_sort(k, descending=descending))
    ko, vo = sort_pairs(g.to_dev(k), g.to_dev(v), n, kdt, np.uint32, descending=descending)
    rk, rv = o.radix_sort(k, v, descending=descending)
    assert same_bits(g.to_host(ko), rk) and same_bits(g.to_host(vo), rv)


# ---------------------------------------------------------------- LDS lane order
@pytest.mark.parametrize("pattern", [0, 1, 2, 3])
def test_lds_atomic_lane_order_probe(gpu, pattern):
    """The stable ranking relies on gfx950 returning same-address LDS atomic
    adds of one instruction in lane order (not an ISA guarantee): a probe over
    uniform, skewed, constant and two-valued digits, 2^24 lane operations
    each, must find no exception."""
    from lc_parallel_primitive_amd import datagen

    log(f"LDS lane-order probe pattern={pattern}")
    assert datagen.lds_order_probe(0x51AB + pattern, pattern, waves=4096, rounds=64) == 0


# ---------------------------------------------------------------- device checkers, pinned
def _mix64(x):
    z = x.astype(np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _host_hash(a):
    with np.errstate(over="ignore"):
        return (int(np.count_nonzero(a[:-1] > a[1:])), int(a.astype(np.uint64).sum(dtype=np.uint64)),
                int(_mix64(a).sum(dtype=np.uint64)))


def test_device_checkers_match_oracle(gpu):
    """The device-side checkers used at sizes above 2^30 agree with the host
    (oracle) checkers, and catch planted mistakes: an adjacent swap, a changed
    key, equal keys whose values are swapped, a value out of range."""
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 100_003
    k = g.random_array(np.uint32, n, seed=77) & np.uint32(0xFFF)
    v = np.arange(n, dtype=np.uint32)
    sk, sv = o.radix_sort(k, v)
    assert datagen.sorted_hash_u32(g.to_dev(k))[1:] == datagen.sorted_hash_u32(g.to_dev(sk))[1:]
    assert datagen.sorted_hash_u32(g.to_dev(sk)) == _host_hash(sk)
    assert datagen.sorted_hash_u32(g.to_dev(sk))[0] == 0
    assert datagen.check_stable_pairs_u32(g.to_dev(k), g.to_dev(sk), g.to_dev(sv)) == 0
    assert o.check_stable_pairs_u64_u32(k.astype(np.uint64), sk.astype(np.uint64), sv)
    i = int(np.flatnonzero(sk[1:] != sk[:-1])[10])  # sk[i] < sk[i+1]
    bad = sk.copy()
    bad[i], bad[i + 1] = bad[i + 1], bad[i]
    assert datagen.sorted_hash_u32(g.to_dev(bad))[0] == 1
    bad = sk.copy()
    bad[5] ^= 1
    assert datagen.sorted_hash_u32(g.to_dev(bad))[1:] != datagen.sorted_hash_u32(g.to_dev(sk))[1:]
    j = int(np.flatnonzero(sk[1:] == sk[:-1])[3])  # equal keys at j, j+1
    bv = sv.copy()
    bv[j], bv[j + 1] = bv[j + 1], bv[j]
    assert datagen.check_stable_pairs_u32(g.to_dev(k), g.to_dev(sk), g.to_dev(bv)) > 0
    assert not o.check_stable_pairs_u64_u32(k.astype(np.uint64), sk.astype(np.uint64), bv)
    bv = sv.copy()
    bv[7] = n
    assert datagen.check_stable_pairs_u32(g.to_dev(k), g.to_dev(sk), g.to_dev(bv)) > 0


# ---------------------------------------------------------------- n >= 2^30
def test_keys_above_2p30(gpu):
    """n = 2^30 + 12345 uint32 keys (the output spans more than 2^32 bytes, so
    the 64-bit write-out path runs): sorted, and the same multiset as the
    input (order-independent sums of the keys and of mix64 of the keys)."""
    import torch

    from lc_parallel_primitive_amd import datagen

    n = (1 << 30) + 12345
    log(f"sort keys u32 n={n}")
    d = datagen.keys_u32(n, seed=0x2B30)
    h_in = datagen.sorted_hash_u32(d)
    out = sort_keys(d, n, np.uint32)
    torch.cuda.synchronize()
    h_out = datagen.sorted_hash_u32(out)
    assert h_out[0] == 0 and h_out[1:] == h_in[1:]
    del d, out


def test_pairs_stable_above_2p30(gpu):
    """n = 2^30 + 777 uint32 keys with 16 random bits (heavy duplication) and
    values = index: the device O(N) stability checker finds no bad position."""
    import torch

    from lc_parallel_primitive_amd import datagen

    n = (1 << 30) + 777
    log(f"sort pairs u32/u32 n={n}")
    k = datagen.keys_u32(n, seed=0x2B31)
    k.view(torch.int32).bitwise_and_(0xFFFF)
    v = datagen.iota_u32(n)
    ko, vo = sort_pairs(k, v, n, np.uint32, np.uint32)
    torch.cuda.synchronize()
    del v
    assert datagen.check_stable_pairs_u32(k, ko, vo) == 0
    del k, ko, vo


def test_keys_at_the_32_bit_limit(gpu):
    """n = 2^32 - 1 uint32 keys, the largest sort that 32-bit positions and
    counts allow (262 144 tiles, the last one a single key short): sorted, the
    same multiset as the input, and a guard region past the output (where
    the last tile's pad would land) untouched."""
    import torch

    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceRadixSort, datagen

    n = (1 << 32) - 1
    guard = 0x5A5A5A5A
    log(f"sort keys u32 n={n}")
    d = datagen.keys_u32(n, seed=0x2B32)
    h_in = datagen.sorted_hash_u32(d)
    buf = torch.full((n + 256,), guard, dtype=torch.int32, device="cuda")
    out = buf.view(torch.uint32)[:n]
    tmp = g.temp(DeviceRadixSort.GetSortKeysTempStorageBytes("uint32", n))
    DeviceRadixSort().SortKeys(tmp, d, out, n)
    torch.cuda.synchronize()
    del d, tmp
    h_out = datagen.sorted_hash_u32(out)
    assert h_out[0] == 0 and h_out[1:] == h_in[1:]
    assert bool((buf[n:] == guard).all())
    del buf, out
    torch.cuda.empty_cache()
