"""Warp- and block-level known answers of the reference
(tests/warp_level_test.cpp:69-239, tests/block_level_test.cpp:67-189),
restated for wave64.  The wave cases run the shared primitives the kernels
are built from (DPP reduce and scans, the segmented (flag, value) scan,
ballot ranks) through datagen.hip's wave_kat kernel; the block cases run the
product's reduce and scan on one 1024-item block (256 threads x 4 items in
the reference), the single-tile path of the device primitives.  Expected
values come from numpy."""
import numpy as np
import pytest

from conftest import log

pytestmark = pytest.mark.gpu

WAVE = 64


def wrap32(a):
    return np.asarray(a, dtype=np.int64).astype(np.uint64).astype(np.uint32).view(np.int32)


def per_wave(a):
    return a.reshape(-1, WAVE)


def seg_cumsum(x, heads):
    """Inclusive sums restarting at every flagged element and every wave start."""
    out = np.empty(x.size, dtype=np.int64)
    acc = 0
    for i in range(x.size):
        if i % WAVE == 0 or heads[i]:
            acc = 0
        acc += int(x[i])
        out[i] = acc
    return wrap32(out)


def cases():
    # the reference's input (i for i < 512), then random data with random flags
    rng = np.random.default_rng(5)
    yield "iota", np.arange(512, dtype=np.int32), None
    yield "random", rng.integers(-(1 << 20), 1 << 20, size=64 * 300, dtype=np.int32), rng.random(64 * 300) < 0.1


@pytest.mark.parametrize("name,x,flags", list(cases()), ids=["iota", "random"])
def test_wave_reductions_and_scans(gpu, name, x, flags):
    # test_warp_reduce (per-warp sum of i) and test_warp_ex_scan (per-warp
    # exclusive sum), plus inclusive sum, inclusive max, min and the lane shift
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    log(f"wave kat reductions/scans {name} n={x.size}")
    d = g.to_dev(x)
    w = per_wave(x.astype(np.int64))
    assert (g.to_host(datagen.wave_kat("reduce_sum", d)) == wrap32(w.sum(axis=1))).all()
    assert (g.to_host(datagen.wave_kat("reduce_min", d)) == w.min(axis=1)).all()
    inc = np.cumsum(w, axis=1)
    assert (g.to_host(datagen.wave_kat("inclusive_sum", d)) == wrap32(inc.ravel())).all()
    assert (g.to_host(datagen.wave_kat("exclusive_sum", d)) == wrap32((inc - w).ravel())).all()
    assert (g.to_host(datagen.wave_kat("inclusive_max", d)) == np.maximum.accumulate(w, axis=1).ravel()).all()
    shifted = np.concatenate([np.full((w.shape[0], 1), -1), w[:, :-1]], axis=1)
    assert (g.to_host(datagen.wave_kat("shift_up", d)) == shifted.ravel()).all()
    if name == "iota":  # the reference's own figures, restated: wave k sums 64k .. 64k + 63
        k = np.arange(x.size // WAVE)
        assert (g.to_host(datagen.wave_kat("reduce_sum", d)) == 64 * 64 * k + 2016).all()


def test_wave_tail_segmented_sum(gpu):
    # test_warp_segment_reduce: values i, a segment ending at every 10th
    # item (key 1 on its last item) and at every warp end; each segment's
    # total equals the sum of its items.  Here the segmented scan of
    # (head, value) pairs: heads follow each tail, and the scan value at a
    # segment's last lane is its total.
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    n = 640
    x = np.arange(n, dtype=np.int32)
    tails = (np.arange(n) % 10) == 9
    heads = np.zeros(n, dtype=bool)
    heads[1:] = tails[:-1]
    log("wave kat tail-segmented sum")
    got = g.to_host(datagen.wave_kat("segmented_sum", g.to_dev(x), g.to_dev(heads.astype(np.int32))))
    assert (got == seg_cumsum(x, heads)).all()
    start = 0
    for i in range(1, n + 1):  # segment boundaries: every 10 items and every wave
        if i == n or i % 10 == 0 or i % WAVE == 0:
            assert got[i - 1] == x[start:i].sum(), (start, i)
            start = i


def test_wave_segmented_sum_random_flags(gpu):
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    rng = np.random.default_rng(9)
    n = 64 * 500
    x = rng.integers(-(1 << 20), 1 << 20, size=n, dtype=np.int32)
    for p in (0.02, 0.3, 1.0):
        heads = rng.random(n) < p
        log(f"wave kat segmented sum p={p}")
        got = g.to_host(datagen.wave_kat("segmented_sum", g.to_dev(x), g.to_dev(heads.astype(np.int32))))
        assert (got == seg_cumsum(x, heads)).all()


def test_wave_flag_rank(gpu):
    # rank among the flagged lanes (the ballot + mbcnt step of the sort's
    # hot-digit ranking and the segment ends' bitmaps)
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen

    rng = np.random.default_rng(13)
    n = 64 * 200
    flags = rng.random(n) < 0.4
    flags[:64] = True  # a full wave
    flags[64:128] = False  # an empty one
    log("wave kat flag rank")
    got = g.to_host(datagen.wave_kat("flag_rank", g.to_dev(np.zeros(n, np.int32)), g.to_dev(flags.astype(np.int32))))
    f = per_wave(flags.astype(np.int64))
    assert (got == (np.cumsum(f, axis=1) - f).ravel()).all()


def test_wave_kat_argument_errors(gpu):
    import torch
    from lc_parallel_primitive_amd import datagen

    L = datagen.lib()
    x = torch.zeros(128, dtype=torch.int32, device="cuda")
    p = x.data_ptr()
    assert L.lcpp_dg_wave_kat(0, p, None, p, 100, None) == -1  # not a multiple of 64
    assert L.lcpp_dg_wave_kat(8, p, None, p, 128, None) == -1  # no such case
    assert L.lcpp_dg_wave_kat(3, p, None, p, 128, None) == -1  # flags needed


# ------------------------------------------------------------------ block level
BLOCK_ITEMS = 256 * 4  # the reference's BLOCKSIZE x ITEMS_PER_THREAD


def test_block_reduce_kat(gpu):
    # test_block_reduce: input i for i < 2000, one sum per 1024-item block
    # (the reference checks the full block: 523776); the partial block too
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceReduce

    x = np.arange(2000, dtype=np.int32)
    d = g.to_dev(x)
    r = DeviceReduce()
    for b0 in range(0, x.size, BLOCK_ITEMS):
        m = min(BLOCK_ITEMS, x.size - b0)
        log(f"block reduce kat block at {b0}, {m} items")
        out = g.empty(1, np.int32)
        tmp = g.temp(DeviceReduce.GetTempStorageBytes("int32", m))
        r.Sum(tmp, d[b0:], out, m)
        assert int(g.to_host(out)[0]) == int(x[b0:b0 + m].sum())
    assert int(x[:BLOCK_ITEMS].sum()) == 523776


@pytest.mark.parametrize("inclusive", [False, True])
def test_block_scan_kat(gpu, inclusive):
    # test_exlusive_scan / test_inlusive_scan: input i, scanned per
    # 1024-item block (the reference asserts the inclusive case only)
    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceScan

    x = np.arange(2000, dtype=np.int32)
    d = g.to_dev(x)
    s = DeviceScan()
    for b0 in range(0, x.size, BLOCK_ITEMS):
        m = min(BLOCK_ITEMS, x.size - b0)
        log(f"block scan kat inclusive={inclusive} block at {b0}")
        out = g.empty(m, np.int32)
        tmp = g.temp(DeviceScan.GetTempStorageBytes("int32", m))
        (s.InclusiveSum if inclusive else s.ExclusiveSum)(tmp, d[b0:], out, m)
        blk = x[b0:b0 + m].astype(np.int64)
        exp = np.cumsum(blk) if inclusive else np.cumsum(blk) - blk
        assert (g.to_host(out) == exp.astype(np.int32)).all()
