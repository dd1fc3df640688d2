"""CPU-side checks of the C ABI boundary: the HIP library loads without a GPU,
exports every symbol include/lcpp_amd.h declares, its size queries are pure
host arithmetic, and argument validation rejects bad calls before any launch."""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "lcpp_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lcpp_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    import lc_parallel_primitive_amd as lcpp

    return lcpp.lib()


def test_every_declared_symbol_is_exported(L):
    names = declared_functions()
    assert len(names) >= 18
    out = subprocess.run(["nm", "-D", "--defined-only", L._name], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (lcpp_[a-z0-9_]+)$", out, flags=re.M))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:  # and ctypes resolves them
        getattr(L, n)


def test_bindings_cover_header():
    from lc_parallel_primitive_amd._capi import SIGNATURES

    assert set(SIGNATURES) == set(declared_functions())


def test_version_and_status_strings(L):
    assert L.lcpp_version() == 100
    assert L.lcpp_status_string(0) == b"LCPP_OK"
    assert L.lcpp_status_string(-2) == b"LCPP_ERR_TEMP_TOO_SMALL"
    assert L.lcpp_status_string(-99) == b"LCPP_ERR_UNKNOWN"


def _q(fn, *args):
    out = ctypes.c_size_t(12345)
    rc = fn(*args, ctypes.byref(out))
    return rc, out.value


# every temp layout starts with the 256-byte status header (lcpp_temp_status)
HDR = 256


def test_temp_bytes_queries(L):
    # reduce: one partial per workgroup (<= 512; <= 1024 for arg), none when one workgroup suffices
    assert _q(L.lcpp_reduce_temp_bytes, 0, 0) == (0, 0)
    assert _q(L.lcpp_reduce_temp_bytes, 0, 8192) == (0, 0)
    rc, b = _q(L.lcpp_reduce_temp_bytes, 0, 1 << 28)  # one partial per workgroup, at most 512
    assert rc == 0 and b == HDR + 512 * 4
    rc, b = _q(L.lcpp_reduce_temp_bytes, 5, 1 << 28)
    assert rc == 0 and b == HDR + 512 * 8
    assert _q(L.lcpp_reduce_temp_bytes, 0, 32768) == (0, 0)  # one 128 KiB tile: one workgroup, no temp
    assert _q(L.lcpp_reduce_temp_bytes, 0, 32769) == (0, HDR + 256)
    # arg reduce: one (value, index) partial per workgroup
    rc, b = _q(L.lcpp_reduce_arg_temp_bytes, 2, 1 << 28)
    assert rc == 0 and b == HDR + 1024 * 8
    rc, b = _q(L.lcpp_reduce_arg_temp_bytes, 5, 1 << 28)
    assert rc == 0 and b == HDR + 1024 * 16
    assert _q(L.lcpp_reduce_arg_temp_bytes, 0, 100) == (0, 0)
    # scan: one packed 64-bit word per tile (two for 64-bit types), counted for
    # the smaller of the exclusive (20480 / 10240) and inclusive (16384 / 8192;
    # 24576 for float) integer tiles
    rc, b = _q(L.lcpp_scan_temp_bytes, 1, 1 << 28)
    assert rc == 0 and b == HDR + (1 << 14) * 8
    rc, b = _q(L.lcpp_scan_temp_bytes, 4, 1 << 27)
    assert rc == 0 and b == HDR + (1 << 14) * 16
    assert _q(L.lcpp_scan_temp_bytes, 1, 0) == (0, 0)
    # sort: header + bins + hot digits + plan + arrival counter, then 4 regions
    # of 16-bit tile counts and 4 of 64-bit batch words + key scratch (no value
    # scratch for keys-only); 16384-key tiles (8192 with values), batches of 8
    rc, b = _q(L.lcpp_radix_sort_keys_temp_bytes, 1, 1 << 28)
    tiles = (1 << 28) // 16384
    head = (HDR + 4 * 256 * 4 + (2 * 4 + 1) * 4 + 255) // 256 * 256
    assert rc == 0 and b == head + 4 * tiles * 256 * 2 + 4 * (tiles // 8) * 256 * 8 + (1 << 28) * 4
    rc, bp = _q(L.lcpp_radix_sort_pairs_temp_bytes, 4, 1, 1 << 27)
    tiles = (1 << 27) // 8192
    head = (HDR + 8 * 256 * 4 + (2 * 8 + 1) * 4 + 255) // 256 * 256
    assert rc == 0 and bp == head + 4 * tiles * 256 * 2 + 4 * (tiles // 8) * 256 * 8 + (1 << 27) * 12
    # the sort takes n up to 2^32 - 1 (32-bit look-back counts and positions)
    rc, b = _q(L.lcpp_radix_sort_keys_temp_bytes, 1, (1 << 32) - 1)
    assert rc == 0 and b > ((1 << 32) - 1) * 4
    # scan by key: one packed word per 8192-value tile (two for 8-byte values)
    rc, b = _q(L.lcpp_scan_by_key_temp_bytes, 0, 2, 1 << 28)
    assert rc == 0 and b == HDR + (1 << 15) * 8
    rc, b = _q(L.lcpp_scan_by_key_temp_bytes, 2, 5, 1 << 27)
    assert rc == 0 and b == HDR + (1 << 15) * 16
    # reduce by key: look-back words per group of 64 tiles and per tile
    # (count, fold), run-count words per batch of 8 tiles (128 bytes each),
    # per-tile summaries (count word, fold), then the dense run slots (128
    # (key, value) entries per tile); each part 256-byte aligned
    def rbk(kb, vb, n, tile):
        tiles = -(-n // tile)
        groups = -(-tiles // 64)
        batches = -(-tiles // 8)
        up = lambda x: -(-x // 256) * 256
        lbw = 1 if vb == 4 else 2
        return (HDR + up(groups * 8) + up(groups * 8 * lbw) + up(tiles * 8) + up(tiles * 8 * lbw) + up(batches * 128)
                + up(tiles * 4) + up(tiles * vb) + up(tiles * 128 * kb) + up(tiles * 128 * vb))
    rc, b = _q(L.lcpp_reduce_by_key_temp_bytes, 0, 0, 1 << 28)
    assert rc == 0 and b == rbk(4, 4, 1 << 28, 8192)
    rc, b = _q(L.lcpp_reduce_by_key_temp_bytes, 5, 5, 100)
    assert rc == 0 and b == rbk(8, 8, 100, 4096)
    rc, b = _q(L.lcpp_reduce_by_key_temp_bytes, 3, 2, 300_000)
    assert rc == 0 and b == rbk(8, 4, 300_000, 8192)
    assert _q(L.lcpp_reduce_by_key_temp_bytes, 0, 9, 100)[0] == -3
    # segment reduce needs none (as the reference)
    assert _q(L.lcpp_segment_reduce_temp_bytes, 2, 1 << 20) == (0, 0)


def test_unsupported_dtype_and_null_args(L):
    assert _q(L.lcpp_reduce_temp_bytes, 17, 10)[0] == -3
    assert L.lcpp_reduce_temp_bytes(0, 10, None) == -1
    # argument errors are detected before any HIP call (no GPU here)
    assert L.lcpp_reduce_sum(9, None, 0, None, None, 10, None) == -3
    assert L.lcpp_reduce_sum(0, None, 0, None, None, 10, None) == -1
    assert L.lcpp_reduce_argmin(0, None, 0, None, None, None, 10, None) == -1
    assert L.lcpp_reduce_argmax(9, None, 0, None, None, None, 10, None) == -3
    one = ctypes.c_int(1)
    assert L.lcpp_reduce_transform(0, 0, 0, None, 0, None, None, 10, None, None) == -1  # init missing
    assert L.lcpp_reduce_transform(0, 7, 0, None, 0, None, None, 10, ctypes.byref(one), None) == -1  # bad op
    assert L.lcpp_reduce_transform(0, 0, 9, None, 0, None, None, 10, ctypes.byref(one), None) == -1  # bad transform
    assert L.lcpp_scan_exclusive_sum(0, None, 0, None, None, 10, None) == -1
    dummy = ctypes.c_void_p(0x1000)
    assert L.lcpp_scan_exclusive(0, 7, dummy, 1 << 20, dummy, dummy, 10, None, None) == -1  # bad op
    assert L.lcpp_scan_inclusive(9, 0, dummy, 1 << 20, dummy, dummy, 10, None, None) == -3
    assert L.lcpp_scan_inclusive(0, 1, None, 0, None, None, 10, None, None) == -1
    assert L.lcpp_scan_exclusive(0, 2, None, 0, None, None, 0, None, None) == 0  # n = 0: nothing to do
    assert L.lcpp_radix_sort_keys(1, None, 0, None, None, 10, None) == -1
    assert L.lcpp_radix_sort_keys(1, None, 0, None, None, 1 << 30, None) == -1  # no temp
    dummy = ctypes.c_void_p(0x1000)
    assert L.lcpp_radix_sort_keys(1, dummy, 1 << 40, dummy, dummy, 1 << 32, None) == -1  # n >= 2^32
    assert L.lcpp_radix_sort_keys_descending(1, None, 0, None, None, 10, None) == -1
    assert L.lcpp_radix_sort_pairs_descending(1, 9, None, 0, None, None, None, None, 10, None) == -3
    assert L.lcpp_radix_sort_pairs_descending(4, 1, None, 0, None, None, None, None, 10, None) == -1
    assert L.lcpp_segment_reduce_sum(2, None, 0, None, None, 10, None, None, None) == -1
    dummy = ctypes.c_void_p(0x1000)
    assert L.lcpp_segment_reduce(2, 5, None, 0, dummy, dummy, 10, dummy, dummy, None, None) == -1  # bad op
    assert L.lcpp_segment_reduce(9, 0, None, 0, dummy, dummy, 10, dummy, dummy, None, None) == -3
    assert L.lcpp_segment_reduce_fixed(0, 0, None, 0, dummy, dummy, 1 << 20, 1 << 12, None, None) == -1  # >= 2^32
    assert L.lcpp_segment_reduce_argmin(0, None, 0, dummy, dummy, None, 10, dummy, dummy, None) == -1  # no index_out
    assert L.lcpp_segment_reduce_argmax_fixed(9, None, 0, dummy, dummy, dummy, 10, 4, None) == -3
    assert _q(L.lcpp_segment_reduce_arg_temp_bytes, 2, 1 << 27, 1 << 20) == (0, 0)
    assert L.lcpp_scan_exclusive_by_key(0, 0, 0, None, 0, None, None, None, 10, None, None) == -1
    assert L.lcpp_scan_inclusive_by_key(0, 0, 5, None, 0, None, None, None, 10, None, None) == -1  # bad op
    assert L.lcpp_scan_inclusive_sum_by_key(9, 0, None, 0, None, None, None, 10, None) == -3
    assert L.lcpp_scan_exclusive_sum_by_key(0, 9, None, 0, None, None, None, 10, None) == -3
    assert L.lcpp_reduce_by_key(0, 0, 0, None, 0, None, None, None, None, None, 10, None) == -1
    assert L.lcpp_reduce_by_key(0, 0, 7, None, 0, None, None, None, None, None, 10, None) == -1
    assert L.lcpp_reduce_by_key(0, 9, 0, None, 0, None, None, None, None, None, 10, None) == -3
    # zero-sized work is a no-op success
    assert L.lcpp_scan_inclusive_sum(0, None, 0, None, None, 0, None) == 0
    assert L.lcpp_radix_sort_keys(1, None, 0, None, None, 0, None) == 0
    assert L.lcpp_segment_reduce_sum(2, None, 0, None, None, 0, None, None, None) == 0
    assert L.lcpp_scan_exclusive_sum_by_key(0, 0, None, 0, None, None, None, 0, None) == 0


def test_temp_too_small_detected_before_launch(L):
    dummy = ctypes.c_void_p(0x1000)
    assert L.lcpp_scan_exclusive_sum(1, dummy, 16, dummy, dummy, 1 << 20, None) == -2
    assert L.lcpp_radix_sort_keys(1, dummy, 16, dummy, dummy, 1 << 20, None) == -2
    assert L.lcpp_reduce_sum(0, dummy, 16, dummy, dummy, 1 << 28, None) == -2
    assert L.lcpp_scan_inclusive_sum_by_key(0, 0, dummy, 16, dummy, dummy, dummy, 1 << 20, None) == -2
    assert L.lcpp_reduce_by_key(0, 0, 0, dummy, 16, dummy, dummy, dummy, dummy, dummy, 1 << 20, None) == -2
    assert L.lcpp_reduce_by_key(0, 0, 0, dummy, 1 << 30, dummy, dummy, dummy, dummy, dummy, 1 << 32, None) == -1


def test_device_status_decode_and_hooks(L):
    # the status word's bits map to status codes without a GPU
    assert L.lcpp_device_status_decode(0) == 0
    assert L.lcpp_device_status_decode(1) == -5
    assert L.lcpp_device_status_decode(0x80000001) == -5
    assert L.lcpp_status_string(-5) == b"LCPP_ERR_LOOKBACK_TIMEOUT"
    assert L.lcpp_test_set_lookback_fault(3, 16) == 0
    assert L.lcpp_test_set_lookback_fault(0xFFFFFFFF, 0) == 0  # back to the defaults
    # the sort's rank-path override: 0 (probe), 1 (LDS atomics), 2 (ballot match)
    assert L.lcpp_test_set_sort_rank_path(3) == -1 and L.lcpp_test_set_sort_rank_path(-1) == -1
    assert L.lcpp_test_set_sort_rank_path(2) == 0 and L.lcpp_test_set_sort_rank_path(0) == 0
    assert L.lcpp_radix_sort_rank_path(None) == -1
    assert L.lcpp_temp_status_record(None, 0, None, None) == -1  # no destination
    dummy = ctypes.c_void_p(0x1000)
    assert L.lcpp_temp_status_record(None, 0, dummy, None) == 0  # no temp: nothing to record, no launch
    assert L.lcpp_temp_status_record(dummy, 255, dummy, None) == 0


def test_misaligned_temp_rejected(L):
    p = ctypes.c_void_p(0x1000 + 4)
    _, b = _q(L.lcpp_scan_temp_bytes, 1, 1 << 20)
    assert L.lcpp_scan_exclusive_sum(1, p, b, p, p, 1 << 20, None) == -1


CPP_USE = r"""
#include "lcpp/parallel_primitive.h"
using namespace luisa::parallel_primitive;
int main()
{
    CommandList cl{};
    BufferView<uint> temp{};
    BufferView<int> ki{}, ko{}, vi{}, vo{};
    BufferView<float> fi{}, fo{};
    BufferView<uint> runs{}, idx{}, beg{}, end{};
    DeviceReduce<> r;
    r.Sum(cl, temp, vi, vo, 10);
    r.Min(cl, temp, vi, vo, 10);
    r.Max(cl, temp, vi, vo, 10);
    r.ArgMin(cl, temp, vi, vo, idx, 10);
    r.ArgMax(cl, temp, vi, vo, idx, 10);
    r.TransformReduce(cl, temp, fi, fo, 10, SumOp{}, SquareOp{}, 0.f);
    r.ReduceByKey(cl, temp, ki, fi, ko, fo, runs, MaxOp{}, 10);
    DeviceScan<> s;
    s.ExclusiveSum(cl, temp, vi, vo, 10);
    s.InclusiveSum(cl, temp, fi, fo, 10);
    s.ExclusiveScanByKey(cl, temp, ki, fi, fo, MinOp{}, 10, 1.f);
    s.InclusiveScanByKey(cl, temp, ki, vi, vo, SumOp{}, 10, 0);
    s.ExclusiveSumByKey(cl, temp, ki, vi, vo, 10);
    s.InclusiveSumByKey(cl, temp, ki, vi, vo, 10);
    DeviceRadixSort<> rs;
    rs.SortKeys(cl, temp, ki, ko, 10u);
    rs.SortPairs(cl, temp, ki, ko, fi, fo, 10u);
    rs.SortKeysDescending(cl, temp, ki, ko, 10u);
    rs.SortPairsDescending(cl, temp, ki, ko, fi, fo, 10u);
    DeviceSegmentReduce<> sr;
    sr.Sum(cl, temp, fi, fo, 10u, beg, end);
    sr.Sum(cl, temp, vi, vo, 10u, 32u);
    sr.Min(cl, temp, fi, fo, 10u, beg, end);
    sr.Max(cl, temp, vi, vo, 10u, 32u);
    sr.Reduce(cl, temp, fi, fo, 10u, beg, end, MaxOp{}, 0.f);
    sr.Reduce(cl, temp, vi, vo, 10u, 7u, SumOp{}, 3);
    sr.ArgMax(cl, temp, fi, fo, idx, 10u, beg, end);
    sr.ArgMax(cl, temp, fi, fo, idx, 10u, 32u);
    sr.ArgMin(cl, temp, vi, vo, idx, 10u, beg, end);
    sr.Argmin(cl, temp, vi, vo, idx, 10u, beg, end);
    sr.ArgMin(cl, temp, vi, vo, idx, 10u, 32u);
    return (int)(DeviceReduce<>::GetTempStorageBytes<int>(10) + DeviceScan<>::GetScanByKeyTempStorageBytes<int, float>(10) +
                 DeviceReduce<>::GetReduceByKeyTempStorageBytes<int, float>(10) +
                 DeviceRadixSort<>::GetSortPairsTempStorageBytes<int, float>(10u) +
                 DeviceSegmentReduce<>::GetTempStorageBytes<float>(10) +
                 DeviceSegmentReduce<>::GetArgTempStorageBytes<float>(10, 2));
}
"""


def test_cpp_host_api_compiles():
    """include/lcpp/parallel_primitive.h (the reference's class names over the
    C ABI) is valid C++17 and every method template instantiates."""
    src = CPP_USE
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                        "-x", "c++", "-"], input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_c_header_is_plain_c():
    src = '#include "lcpp_amd.h"\nint main(void){return lcpp_version();}\n'
    r = subprocess.run(["gcc", "-std=c99", "-fsyntax-only", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                        "-x", "c", "-"], input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
