"""Device status word (lcpp_temp_status, the counterpart of the reference's
debug-stream lcpp_check, runtime/core.h:56-64): a decoupled look-back wait that
gives up is reported, not silent.

The give-up is forced from the host with the test hook
lcpp_test_set_lookback_fault: one tile never publishes its look-back words and
waits give up after a few re-polls.  Every kernel still drains and every access
stays in bounds (positions are range-checked); the outputs of those calls are
wrong by design and are not compared.  A normal call on the same temp storage
afterwards must report LCPP_OK again and be exact."""
import ctypes
from contextlib import contextmanager

import numpy as np
import pytest

from conftest import log
from oracle import oracle as o

pytestmark = pytest.mark.gpu

OK, TIMEOUT = 0, -5


def _L():
    import lc_parallel_primitive_amd as lcpp

    return lcpp.lib()


def _sp():
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


@contextmanager
def withheld(tile, spins=32):
    L = _L()
    assert L.lcpp_test_set_lookback_fault(tile, spins) == 0
    try:
        yield
    finally:
        L.lcpp_test_set_lookback_fault(0xFFFFFFFF, 0)


def status(temp):
    return _L().lcpp_temp_status(_p(temp), temp.numel(), _sp())


def _temp(fn, *args):
    import gpu_util as g

    b = ctypes.c_size_t()
    assert fn(*args, ctypes.byref(b)) == 0
    return g.temp(b.value)


def test_scan_withheld_tile_reports_timeout(gpu):
    import gpu_util as g

    L = _L()
    n = 1 << 20  # 52 exclusive tiles of 20480
    a = g.random_array(np.uint32, n, seed=1)
    d, out = g.to_dev(a), g.empty(n, np.uint32)
    t = _temp(L.lcpp_scan_temp_bytes, 1, n)
    log("status: scan with tile 3 withheld")
    with withheld(3):
        assert L.lcpp_scan_exclusive_sum(1, _p(t), t.numel(), _p(d), _p(out), n, _sp()) == 0
        assert status(t) == TIMEOUT
    assert L.lcpp_scan_exclusive_sum(1, _p(t), t.numel(), _p(d), _p(out), n, _sp()) == 0
    assert status(t) == OK
    assert (g.to_host(out) == o.scan(a, inclusive=False)).all()


@pytest.mark.parametrize("pairs", [False, True])
def test_sort_withheld_tile_reports_timeout(gpu, pairs):
    import gpu_util as g

    L = _L()
    n = 40 * 16384 + 5  # 5+ look-back batches of 16384-key tiles (8192 with values)
    k = g.random_array(np.uint32, n, seed=2)
    v = np.arange(n, dtype=np.uint32)
    dk, dv = g.to_dev(k), g.to_dev(v)
    ko, vo = g.empty(n, np.uint32), g.empty(n, np.uint32)
    if pairs:
        t = _temp(L.lcpp_radix_sort_pairs_temp_bytes, 1, 1, n)
        call = lambda: L.lcpp_radix_sort_pairs(1, 1, _p(t), t.numel(), _p(dk), _p(ko), _p(dv), _p(vo), n, _sp())
    else:
        t = _temp(L.lcpp_radix_sort_keys_temp_bytes, 1, n)
        call = lambda: L.lcpp_radix_sort_keys(1, _p(t), t.numel(), _p(dk), _p(ko), n, _sp())
    for tile in (0, 9, 23):  # a batch's first tile, a middle one, a batch's last (its inclusive prefix)
        log(f"status: sort pairs={pairs} tile {tile} withheld")
        with withheld(tile):
            assert call() == 0
            assert status(t) == TIMEOUT
    assert call() == 0
    assert status(t) == OK
    if pairs:
        rk, rv = o.radix_sort(k, v)
        assert (g.to_host(ko) == rk).all() and (g.to_host(vo) == rv).all()
    else:
        assert (g.to_host(ko) == o.radix_sort(k)).all()


def test_status_record_accumulates_without_synchronizing(gpu):
    """lcpp_temp_status_record ORs each call's status word into a caller word
    on the stream: three sorts (normal, one with a withheld tile, normal again)
    leave the bit set in the accumulated word, a clean word stays 0, and
    a call without temp storage records nothing."""
    import torch

    import gpu_util as g

    L = _L()
    n = 20 * 16384 + 3
    k = g.random_array(np.uint32, n, seed=5)
    dk, ko = g.to_dev(k), g.empty(n, np.uint32)
    t = _temp(L.lcpp_radix_sort_keys_temp_bytes, 1, n)
    acc = torch.zeros(1, dtype=torch.int32, device="cuda")
    clean = torch.zeros(1, dtype=torch.int32, device="cuda")
    log("status record: three sorts, the second with tile 7 withheld")
    assert L.lcpp_radix_sort_keys(1, _p(t), t.numel(), _p(dk), _p(ko), n, _sp()) == 0
    assert L.lcpp_temp_status_record(_p(t), t.numel(), _p(acc), _sp()) == 0
    assert L.lcpp_temp_status_record(_p(t), t.numel(), _p(clean), _sp()) == 0
    with withheld(7):
        assert L.lcpp_radix_sort_keys(1, _p(t), t.numel(), _p(dk), _p(ko), n, _sp()) == 0
        assert L.lcpp_temp_status_record(_p(t), t.numel(), _p(acc), _sp()) == 0
    assert L.lcpp_radix_sort_keys(1, _p(t), t.numel(), _p(dk), _p(ko), n, _sp()) == 0
    assert L.lcpp_temp_status_record(_p(t), t.numel(), _p(acc), _sp()) == 0
    assert L.lcpp_temp_status_record(None, 0, _p(acc), _sp()) == 0  # no temp: nothing recorded
    assert L.lcpp_temp_status_record(_p(t), t.numel(), None, _sp()) == -1
    torch.cuda.synchronize()
    word = int(acc.item()) & 0xFFFFFFFF
    assert word & 1 and L.lcpp_device_status_decode(word) == TIMEOUT
    assert int(clean.item()) == 0
    assert (g.to_host(ko) == o.radix_sort(k)).all()  # the last call was a normal one


def test_by_key_withheld_tile_reports_timeout(gpu):
    import gpu_util as g

    L = _L()
    n = 300_000  # ~37 tiles of 8192
    keys = (np.arange(n) // 97).astype(np.int32)
    vals = g.random_array(np.int32, n, seed=3)
    dk, dv = g.to_dev(keys), g.to_dev(vals)
    out = g.empty(n, np.int32)
    t = _temp(L.lcpp_scan_by_key_temp_bytes, 0, 0, n)
    log("status: scan by key tile 4 withheld")
    with withheld(4):
        assert L.lcpp_scan_inclusive_sum_by_key(0, 0, _p(t), t.numel(), _p(dk), _p(dv), _p(out), n, _sp()) == 0
        assert status(t) == TIMEOUT
    assert L.lcpp_scan_inclusive_sum_by_key(0, 0, _p(t), t.numel(), _p(dk), _p(dv), _p(out), n, _sp()) == 0
    assert status(t) == OK
    assert (g.to_host(out) == o.scan_by_key(keys, vals, inclusive=True)).all()

    # ReduceByKey's look-back runs over groups of 64 tiles (its emit launch):
    # withhold group 4 of 7
    n = 7 * 64 * 8192 - 1000
    keys = (np.arange(n) // 97).astype(np.int32)
    vals = g.random_array(np.int32, n, seed=5)
    dk, dv = g.to_dev(keys), g.to_dev(vals)
    uk, agg, runs = g.empty(n, np.int32), g.empty(n, np.int32), g.empty(1, np.uint32)
    t = _temp(L.lcpp_reduce_by_key_temp_bytes, 0, 0, n)
    log("status: reduce by key group 4 withheld")
    with withheld(4):
        assert L.lcpp_reduce_by_key(0, 0, 0, _p(t), t.numel(), _p(dk), _p(dv), _p(uk), _p(agg), _p(runs), n,
                                    _sp()) == 0
        assert status(t) == TIMEOUT
    assert L.lcpp_reduce_by_key(0, 0, 0, _p(t), t.numel(), _p(dk), _p(dv), _p(uk), _p(agg), _p(runs), n, _sp()) == 0
    assert status(t) == OK
    ek, ev = o.reduce_by_key(keys, vals)
    r = int(g.to_host(runs)[0])
    assert r == ek.size and (g.to_host(uk)[:r] == ek).all() and (g.to_host(agg)[:r] == ev).all()

    # tiles with more than 128 runs wait in the tile launch itself for the
    # counts of their batch-mates (batches of 8 tiles) and the words of the
    # batches before them: distinct keys, and withheld tile 4 (a batch-mate of
    # tiles 5-7) or tile 15 (batch 1's last tile: batch 1 never completes and
    # never gets the inclusive count that tile would add, so every later
    # tile's walk stalls on its word)
    n = 40 * 8192 + 3
    keys = np.arange(n, dtype=np.int32)
    vals = g.random_array(np.int32, n, seed=6)
    dk, dv = g.to_dev(keys), g.to_dev(vals)
    uk, agg, runs = g.empty(n, np.int32), g.empty(n, np.int32), g.empty(1, np.uint32)
    t = _temp(L.lcpp_reduce_by_key_temp_bytes, 0, 0, n)
    for tile in (4, 15):
        log(f"status: reduce by key, dense tiles, tile {tile} withheld")
        with withheld(tile):
            assert L.lcpp_reduce_by_key(0, 0, 0, _p(t), t.numel(), _p(dk), _p(dv), _p(uk), _p(agg), _p(runs), n,
                                        _sp()) == 0
            assert status(t) == TIMEOUT
        assert L.lcpp_reduce_by_key(0, 0, 0, _p(t), t.numel(), _p(dk), _p(dv), _p(uk), _p(agg), _p(runs), n,
                                    _sp()) == 0
        assert status(t) == OK
        r = int(g.to_host(runs)[0])
        assert r == n and (g.to_host(uk) == keys).all() and (g.to_host(agg) == vals).all()


def test_status_cleared_by_every_primitive(gpu):
    """A status word left set by an earlier call is cleared by the next call
    that uses the same temp storage, including calls that never wait."""
    import torch

    import gpu_util as g

    L = _L()
    n = 1 << 20
    a = g.random_array(np.int32, n, seed=4)
    d, o1 = g.to_dev(a), g.empty(1, np.int32)
    idx = g.empty(1, np.uint32)
    t = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    for name, call in [
        ("reduce", lambda: L.lcpp_reduce_sum(0, _p(t), t.numel(), _p(d), _p(o1), n, _sp())),
        ("reduce small", lambda: L.lcpp_reduce_sum(0, _p(t), t.numel(), _p(d), _p(o1), 1000, _sp())),
        ("argmax", lambda: L.lcpp_reduce_argmax(0, _p(t), t.numel(), _p(d), _p(o1), _p(idx), n, _sp())),
        ("scan", lambda: L.lcpp_scan_inclusive_sum(0, _p(t), t.numel(), _p(d), _p(g.empty(n, np.int32)), n, _sp())),
    ]:
        log(f"status cleared by {name}")
        t.fill_(0xFF)
        assert status(t) == TIMEOUT  # the word reads as set
        assert call() == 0
        assert status(t) == OK, name
