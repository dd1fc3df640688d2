"""Calls from several host threads at once, each on its own stream with its
own temp buffer (the C ABI's thread-safety contract: calls that do not share
temp storage may overlap).  Every call's output is checked against the
oracle; the sort's first calls in each thread also race on the library's
per-device launch caches (CU count, occupancy, the histogram's LDS limit)."""
import threading

import numpy as np
import pytest

from conftest import log
from oracle import oracle as o

pytestmark = pytest.mark.gpu

THREADS = 4
ROUNDS = 3


def test_threads_distinct_temp_and_streams(gpu):
    import torch

    import gpu_util as g
    from lc_parallel_primitive_amd import DeviceRadixSort, DeviceReduce, DeviceScan, DeviceSegmentReduce

    n = 200_003
    jobs = []
    for t in range(THREADS):
        k = g.random_array(np.uint32, n, seed=100 + t)
        v = np.arange(n, dtype=np.uint32)
        x = g.random_array(np.int32, n, seed=200 + t)
        seg = np.sort(np.random.default_rng(300 + t).integers(0, n, size=2 * 1000, dtype=np.uint32))
        begin, end = seg[0::2].copy(), seg[1::2].copy()
        jobs.append(dict(
            k=k, v=v, x=x, begin=begin, end=end,
            dk=g.to_dev(k), dv=g.to_dev(v), dx=g.to_dev(x), db=g.to_dev(begin), de=g.to_dev(end),
            ko=g.empty(n, np.uint32), vo=g.empty(n, np.uint32), so=g.empty(n, np.int32),
            ro=g.empty(1, np.int32), go=g.empty(len(begin), np.int32),
            t_sort=g.temp(DeviceRadixSort.GetSortPairsTempStorageBytes("uint32", "uint32", n)),
            t_scan=g.temp(DeviceScan.GetTempStorageBytes("int32", n)),
            t_red=g.temp(DeviceReduce.GetTempStorageBytes("int32", n)),
            stream=torch.cuda.Stream(),
        ))
    torch.cuda.synchronize()
    errors = []

    def work(j):
        try:
            s = j["stream"]
            for _ in range(ROUNDS):
                DeviceRadixSort().SortPairs(j["t_sort"], j["dk"], j["ko"], j["dv"], j["vo"], n, stream=s)
                DeviceScan().InclusiveSum(j["t_scan"], j["dx"], j["so"], n, stream=s)
                DeviceReduce().Sum(j["t_red"], j["dx"], j["ro"], n, stream=s)
                DeviceSegmentReduce().Sum(None, j["dx"], j["go"], len(j["begin"]), j["db"], j["de"], stream=s)
        except Exception as e:  # reported on the main thread
            errors.append(e)

    log(f"concurrency: {THREADS} threads x {ROUNDS} rounds, n={n}")
    threads = [threading.Thread(target=work, args=(j,)) for j in jobs]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for j in jobs:
        rk, rv = o.radix_sort(j["k"], j["v"])
        assert (g.to_host(j["ko"]) == rk).all() and (g.to_host(j["vo"]) == rv).all()
        assert (g.to_host(j["so"]) == np.cumsum(j["x"], dtype=np.int32)).all()
        assert g.to_host(j["ro"])[0] == j["x"].sum(dtype=np.int32)  # wraps mod 2^32
        cs = np.concatenate([[0], np.cumsum(j["x"], dtype=np.int64)])
        want = ((cs[j["end"]] - cs[j["begin"]]) & 0xFFFFFFFF).astype(np.uint32).view(np.int32)
        assert (g.to_host(j["go"]) == want).all()


def test_concurrent_large_sorts(gpu):
    """Four streams each queue four 2^24-key sorts (1024 tiles each, far more
    than one sort's 128-workgroup look-ahead) without waiting in between, so
    the sorts overlap on the GPU: every call's status word must read OK and
    its output must be the sorted permutation of its input."""
    import ctypes

    import torch

    import gpu_util as g
    import lc_parallel_primitive_amd as lcpp
    from lc_parallel_primitive_amd import DeviceRadixSort

    n, rounds = 1 << 24, 4
    L = lcpp.lib()
    tb = DeviceRadixSort.GetSortKeysTempStorageBytes("uint32", n)
    jobs = []
    for t in range(THREADS):
        k = g.random_array(np.uint32, n, seed=400 + t)
        jobs.append(dict(k=k, dk=g.to_dev(k), ko=[g.empty(n, np.uint32) for _ in range(rounds)],
                         temp=[g.temp(tb) for _ in range(rounds)], stream=torch.cuda.Stream()))
    torch.cuda.synchronize()
    errors = []
    barrier = threading.Barrier(THREADS)

    def work(j):
        try:
            barrier.wait()
            for r in range(rounds):
                DeviceRadixSort().SortKeys(j["temp"][r], j["dk"], j["ko"][r], n, stream=j["stream"])
        except Exception as e:  # reported on the main thread
            errors.append(e)

    log(f"concurrency: {THREADS} streams x {rounds} queued SortKeys of n={n}")
    threads = [threading.Thread(target=work, args=(j,)) for j in jobs]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for t, j in enumerate(jobs):
        for r in range(rounds):
            st = L.lcpp_temp_status(ctypes.c_void_p(j["temp"][r].data_ptr()), j["temp"][r].numel(),
                                    ctypes.c_void_p(j["stream"].cuda_stream))
            assert st == 0, (t, r, st)
            assert o.check_sorted_permutation_u32(j["k"], g.to_host(j["ko"][r])), (t, r)
