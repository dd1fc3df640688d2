"""Device-level primitives with the reference's class and method names.

Mirrors src/lcpp/device/device_{reduce,scan,radix_sort,segment_reduce}.h of
the reference: caller-owned temp storage sized by the static
Get*TempStorageBytes queries, then an asynchronous call on a stream.  The
reference records into an LC CommandList; here the work is enqueued on a
HIP stream (default: torch's current stream).  Buffers are device tensors
(torch here; anything with .data_ptr(), .numel(), .element_size(), .dtype).

Differences from the reference, by design:
  * errors raise LcppError (the reference asserts in debug builds and
    ignores failures in release, runtime/core.h:56-67);
  * sizes are checked against the buffers before any launch;
  * DeviceReduce.Max starts from numeric lowest() (the reference uses
    numeric_limits<T>::min(), wrong for floating point,
    device_reduce.h:181-185).
"""
from __future__ import annotations

import ctypes

from ._capi import LCPP_OPS, LCPP_TRANSFORMS, check, dtype_code, lib


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(stream):
    if stream is None:
        import torch

        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return ctypes.c_void_p(stream)
    return ctypes.c_void_p(stream.cuda_stream)


def _nbytes(t) -> int:
    return 0 if t is None else t.numel() * t.element_size()


def _need(t, n: int, what: str):
    if n > 0 and (t is None or t.numel() < n):
        raise ValueError(f"{what}: buffer holds {0 if t is None else t.numel()} elements, need {n}")


def _same_dtype(a, b, what: str):
    if a.dtype != b.dtype:
        raise TypeError(f"{what}: dtype mismatch {a.dtype} vs {b.dtype}")


_NP_DTYPES = ["int32", "uint32", "float32", "int64", "uint64", "float64"]


def _host_value(code: int, value):
    """A one-element numpy array of lcpp_dtype `code` holding `value` (kept
    alive by the caller for the duration of the call)."""
    import numpy as np

    return np.array([value], dtype=_NP_DTYPES[code])


def _query(fn, *args) -> int:
    out = ctypes.c_size_t()
    check(fn(*args, ctypes.byref(out)), fn.__name__)
    return out.value


class _Module:
    """What every module shares.  The geometry arguments are accepted for source
    compatibility (the library fixes it per dtype, tuned for gfx950).

    create(device, debug_stream) follows the reference's modules, whose
    lcpp_check commits, synchronizes and asserts after each step when a debug
    stream is given (runtime/core.h:56-64): here every call is then
    synchronized and the device status word of its temp storage is read
    (lcpp_temp_status), so a look-back wait that gave up raises LcppError
    (LCPP_ERR_LOOKBACK_TIMEOUT) at the call that caused it.  Without a debug
    stream no call synchronizes."""

    def __init__(self, BLOCK_SIZE: int = 256, WARP_NUMS: int = 64, ITEMS_PER_THREAD: int = 16):
        self.geometry = (BLOCK_SIZE, WARP_NUMS, ITEMS_PER_THREAD)
        self._debug = False

    def create(self, device=None, debug_stream=None):
        self._debug = debug_stream is not None
        return self

    def _check(self, status: int, what: str, temp, stream) -> None:
        check(status, what)
        if self._debug:
            check(lib().lcpp_temp_status(_ptr(temp), _nbytes(temp), _stream(stream)), what + " (device status)")


class DeviceReduce(_Module):
    """device/device_reduce.h:37-348 (Sum / Min / Max / ArgMin / ArgMax / ReduceByKey / TransformReduce)."""


    @staticmethod
    def GetTempStorageBytes(dtype, num_item: int) -> int:
        return _query(lib().lcpp_reduce_temp_bytes, dtype_code(dtype), num_item)

    def _run(self, fn, temp, d_in, d_out, num_item, stream):
        _need(d_in, num_item, "d_in")
        _need(d_out, 1, "d_out")
        _same_dtype(d_in, d_out, fn.__name__)
        self._check(fn(dtype_code(d_in.dtype), _ptr(temp), _nbytes(temp), _ptr(d_in), _ptr(d_out), num_item,
                 _stream(stream)), fn.__name__, temp, stream)

    def Sum(self, temp_storage, d_in, d_out, num_item: int, stream=None):
        self._run(lib().lcpp_reduce_sum, temp_storage, d_in, d_out, num_item, stream)

    def Min(self, temp_storage, d_in, d_out, num_item: int, stream=None):
        self._run(lib().lcpp_reduce_min, temp_storage, d_in, d_out, num_item, stream)

    def Max(self, temp_storage, d_in, d_out, num_item: int, stream=None):
        self._run(lib().lcpp_reduce_max, temp_storage, d_in, d_out, num_item, stream)

    @staticmethod
    def GetArgTempStorageBytes(dtype, num_item: int) -> int:
        return _query(lib().lcpp_reduce_arg_temp_bytes, dtype_code(dtype), num_item)

    def _arg(self, fn, temp, d_in, d_out, d_index_out, num_item, stream):
        _need(d_in, num_item, "d_in")
        _need(d_out, 1, "d_out")
        _need(d_index_out, 1, "d_index_out")
        _same_dtype(d_in, d_out, fn.__name__)
        if d_index_out.element_size() != 4:
            raise TypeError(f"{fn.__name__}: d_index_out must hold 32-bit indices")
        self._check(fn(dtype_code(d_in.dtype), _ptr(temp), _nbytes(temp), _ptr(d_in), _ptr(d_out), _ptr(d_index_out),
                 num_item, _stream(stream)), fn.__name__, temp, stream)

    def ArgMin(self, temp_storage, d_in, d_out, d_index_out, num_item: int, stream=None):
        """device_reduce.h:187-227: smallest value, ties to the smallest index."""
        self._arg(lib().lcpp_reduce_argmin, temp_storage, d_in, d_out, d_index_out, num_item, stream)

    def ArgMax(self, temp_storage, d_in, d_out, d_index_out, num_item: int, stream=None):
        """device_reduce.h:229-272: largest value, ties to the largest index (ArgMaxOp)."""
        self._arg(lib().lcpp_reduce_argmax, temp_storage, d_in, d_out, d_index_out, num_item, stream)

    def Reduce(self, temp_storage, d_in, d_out, num_item: int, reduce_op: str, initial_value, stream=None):
        """device_reduce.h:131-147: d_out[0] = reduce_op(initial_value, reduce_op over d_in[0..num_item)).
        reduce_op: "sum" | "min" | "max"."""
        self.TransformReduce(temp_storage, d_in, d_out, num_item, reduce_op, "identity", initial_value, stream)

    def TransformReduce(self, temp_storage, d_in, d_out, num_item: int, reduce_op: str, transform_op: str, init,
                        stream=None):
        """device_reduce.h:331-348: d_out[0] = reduce_op(init, reduce_op over i of transform_op(d_in[i])).
        reduce_op: "sum" | "min" | "max"; transform_op: "identity" | "negate" | "abs" | "square"."""
        import numpy as np

        _need(d_in, num_item, "d_in")
        _need(d_out, 1, "d_out")
        _same_dtype(d_in, d_out, "TransformReduce")
        if reduce_op not in LCPP_OPS or transform_op not in LCPP_TRANSFORMS:
            raise ValueError(f"TransformReduce: unsupported ({reduce_op!r}, {transform_op!r})")
        code = dtype_code(d_in.dtype)
        np_dt = [np.int32, np.uint32, np.float32, np.int64, np.uint64, np.float64][code]
        iv = np.array([init], dtype=np_dt)
        self._check(lib().lcpp_reduce_transform(code, LCPP_OPS[reduce_op], LCPP_TRANSFORMS[transform_op], _ptr(temp_storage),
                                          _nbytes(temp_storage), _ptr(d_in), _ptr(d_out), num_item,
                                          ctypes.c_void_p(iv.ctypes.data), _stream(stream)),
              "lcpp_reduce_transform", temp_storage, stream)

    @staticmethod
    def GetReduceByKeyTempStorageBytes(key_dtype, value_dtype, num_elements: int) -> int:
        """device_reduce.h:110-125"""
        return _query(lib().lcpp_reduce_by_key_temp_bytes, dtype_code(key_dtype), dtype_code(value_dtype),
                      num_elements)

    def ReduceByKey(self, temp_storage, d_keys_in, d_values_in, d_unique_out, g_aggregates_out, g_num_runs_out,
                    reduce_op: str, num_elements: int, stream=None):
        """device_reduce.h:277-318: one (key, op-fold of values) per run of equal consecutive keys;
        g_num_runs_out[0] (a device uint32) = number of runs.  reduce_op: "sum" | "min" | "max"."""
        for t, nm in ((d_keys_in, "d_keys_in"), (d_values_in, "d_values_in"), (d_unique_out, "d_unique_out"),
                      (g_aggregates_out, "g_aggregates_out")):
            _need(t, num_elements, nm)
        _need(g_num_runs_out, 1, "g_num_runs_out")
        _same_dtype(d_keys_in, d_unique_out, "ReduceByKey keys")
        _same_dtype(d_values_in, g_aggregates_out, "ReduceByKey values")
        if g_num_runs_out.element_size() != 4:
            raise TypeError("ReduceByKey: g_num_runs_out must hold a 32-bit count")
        if reduce_op not in LCPP_OPS:
            raise ValueError(f"ReduceByKey: unsupported reduce_op {reduce_op!r}")
        self._check(lib().lcpp_reduce_by_key(dtype_code(d_keys_in.dtype), dtype_code(d_values_in.dtype), LCPP_OPS[reduce_op],
                                       _ptr(temp_storage), _nbytes(temp_storage), _ptr(d_keys_in), _ptr(d_values_in),
                                       _ptr(d_unique_out), _ptr(g_aggregates_out), _ptr(g_num_runs_out), num_elements,
                                       _stream(stream)),
              "lcpp_reduce_by_key", temp_storage, stream)


class DeviceScan(_Module):
    """device/device_scan.h:33-339 (ExclusiveScan / InclusiveScan / ExclusiveSum / InclusiveSum / *ScanByKey /
    *SumByKey)."""


    @staticmethod
    def GetTempStorageBytes(dtype, num_items: int) -> int:
        return _query(lib().lcpp_scan_temp_bytes, dtype_code(dtype), num_items)

    def _run(self, fn, temp, d_in, d_out, num_items, stream):
        _need(d_in, num_items, "d_in")
        _need(d_out, num_items, "d_out")
        _same_dtype(d_in, d_out, fn.__name__)
        self._check(fn(dtype_code(d_in.dtype), _ptr(temp), _nbytes(temp), _ptr(d_in), _ptr(d_out), num_items,
                 _stream(stream)), fn.__name__, temp, stream)

    def ExclusiveSum(self, temp_storage, d_in, d_out, num_items: int, stream=None):
        self._run(lib().lcpp_scan_exclusive_sum, temp_storage, d_in, d_out, num_items, stream)

    def InclusiveSum(self, temp_storage, d_in, d_out, num_items: int, stream=None):
        self._run(lib().lcpp_scan_inclusive_sum, temp_storage, d_in, d_out, num_items, stream)

    def _scan_op(self, fn, name, temp, d_in, d_out, num_items, op, init, stream):
        _need(d_in, num_items, "d_in")
        _need(d_out, num_items, "d_out")
        _same_dtype(d_in, d_out, name)
        if op not in LCPP_OPS:
            raise ValueError(f"{name}: unsupported scan_op {op!r}")
        code = dtype_code(d_in.dtype)
        iv = _host_value(code, init)
        self._check(fn(code, LCPP_OPS[op], _ptr(temp), _nbytes(temp), _ptr(d_in), _ptr(d_out), num_items,
                       ctypes.c_void_p(iv.ctypes.data), _stream(stream)), name, temp, stream)

    def ExclusiveScan(self, temp_storage, d_in, d_out, num_items: int, scan_op: str, initial_value, stream=None):
        """device_scan.h:114-145: out[i] = scan_op(initial_value, d_in[0..i)), out[0] = initial_value.
        scan_op: "sum" | "min" | "max"."""
        self._scan_op(lib().lcpp_scan_exclusive, "ExclusiveScan", temp_storage, d_in, d_out, num_items, scan_op,
                      initial_value, stream)

    def InclusiveScan(self, temp_storage, d_in, d_out, num_items: int, scan_op: str, initial_value, stream=None):
        """device_scan.h:147-178: out[i] = scan_op(initial_value, d_in[0..i])."""
        self._scan_op(lib().lcpp_scan_inclusive, "InclusiveScan", temp_storage, d_in, d_out, num_items, scan_op,
                      initial_value, stream)

    @staticmethod
    def GetScanByKeyTempStorageBytes(key_dtype, value_dtype, num_items: int) -> int:
        """device_scan.h:91-107"""
        return _query(lib().lcpp_scan_by_key_temp_bytes, dtype_code(key_dtype), dtype_code(value_dtype), num_items)

    def _by_key(self, fn, name, temp, d_keys_in, d_values_in, d_values_out, num_items, op, init, stream):
        _need(d_keys_in, num_items, "d_keys_in")
        _need(d_values_in, num_items, "d_values_in")
        _need(d_values_out, num_items, "d_values_out")
        _same_dtype(d_values_in, d_values_out, name)
        if op not in LCPP_OPS:
            raise ValueError(f"{name}: unsupported scan_op {op!r}")
        vcode = dtype_code(d_values_in.dtype)
        iv = _host_value(vcode, init)
        self._check(fn(dtype_code(d_keys_in.dtype), vcode, LCPP_OPS[op], _ptr(temp), _nbytes(temp), _ptr(d_keys_in),
                 _ptr(d_values_in), _ptr(d_values_out), num_items, ctypes.c_void_p(iv.ctypes.data), _stream(stream)),
              name, temp, stream)

    def ExclusiveScanByKey(self, temp_storage, d_keys_in, d_values_in, d_values_out, scan_op: str, num_items: int,
                           initial_value, stream=None):
        """device_scan.h:206-254: runs of equal consecutive keys; out = initial_value at a head, else
        scan_op(fold of the run's earlier values, initial_value).  scan_op: "sum" | "min" | "max"."""
        self._by_key(lib().lcpp_scan_exclusive_by_key, "ExclusiveScanByKey", temp_storage, d_keys_in, d_values_in,
                     d_values_out, num_items, scan_op, initial_value, stream)

    def InclusiveScanByKey(self, temp_storage, d_keys_in, d_values_in, d_values_out, scan_op: str, num_items: int,
                           initial_value, stream=None):
        """device_scan.h:256-303: out = scan_op(fold of the run's values up to i, initial_value)."""
        self._by_key(lib().lcpp_scan_inclusive_by_key, "InclusiveScanByKey", temp_storage, d_keys_in, d_values_in,
                     d_values_out, num_items, scan_op, initial_value, stream)

    def ExclusiveSumByKey(self, temp_storage, d_keys_in, d_values_in, d_values_out, num_items: int, stream=None):
        """device_scan.h:306-322"""
        self.ExclusiveScanByKey(temp_storage, d_keys_in, d_values_in, d_values_out, "sum", num_items, 0, stream)

    def InclusiveSumByKey(self, temp_storage, d_keys_in, d_values_in, d_values_out, num_items: int, stream=None):
        """device_scan.h:324-339"""
        self.InclusiveScanByKey(temp_storage, d_keys_in, d_values_in, d_values_out, "sum", num_items, 0, stream)


class DeviceRadixSort(_Module):
    """device/device_radix_sort.h:37-184 (onesweep SortKeys / SortPairs, ascending and descending)."""


    @staticmethod
    def GetSortKeysTempStorageBytes(key_dtype, num_items: int) -> int:
        return _query(lib().lcpp_radix_sort_keys_temp_bytes, dtype_code(key_dtype), num_items)

    @staticmethod
    def GetSortPairsTempStorageBytes(key_dtype, value_dtype, num_items: int) -> int:
        return _query(lib().lcpp_radix_sort_pairs_temp_bytes, dtype_code(key_dtype), dtype_code(value_dtype),
                      num_items)

    def _keys(self, fn, name, temp_storage, d_keys_in, d_keys_out, num_items, stream):
        _need(d_keys_in, num_items, "d_keys_in")
        _need(d_keys_out, num_items, "d_keys_out")
        _same_dtype(d_keys_in, d_keys_out, name)
        self._check(fn(dtype_code(d_keys_in.dtype), _ptr(temp_storage), _nbytes(temp_storage), _ptr(d_keys_in),
                 _ptr(d_keys_out), num_items, _stream(stream)), name, temp_storage, stream)

    def _pairs(self, fn, name, temp_storage, d_keys_in, d_keys_out, d_values_in, d_values_out, num_items, stream):
        for t, nm in ((d_keys_in, "d_keys_in"), (d_keys_out, "d_keys_out"), (d_values_in, "d_values_in"),
                      (d_values_out, "d_values_out")):
            _need(t, num_items, nm)
        _same_dtype(d_keys_in, d_keys_out, name + " keys")
        _same_dtype(d_values_in, d_values_out, name + " values")
        self._check(fn(dtype_code(d_keys_in.dtype), dtype_code(d_values_in.dtype), _ptr(temp_storage),
                 _nbytes(temp_storage), _ptr(d_keys_in), _ptr(d_keys_out), _ptr(d_values_in), _ptr(d_values_out),
                 num_items, _stream(stream)), name, temp_storage, stream)

    def SortKeys(self, temp_storage, d_keys_in, d_keys_out, num_items: int, stream=None):
        self._keys(lib().lcpp_radix_sort_keys, "lcpp_radix_sort_keys", temp_storage, d_keys_in, d_keys_out,
                   num_items, stream)

    def SortPairs(self, temp_storage, d_keys_in, d_keys_out, d_values_in, d_values_out, num_items: int,
                  stream=None):
        self._pairs(lib().lcpp_radix_sort_pairs, "lcpp_radix_sort_pairs", temp_storage, d_keys_in, d_keys_out,
                    d_values_in, d_values_out, num_items, stream)

    def SortKeysDescending(self, temp_storage, d_keys_in, d_keys_out, num_items: int, stream=None):
        """device_radix_sort.h:172-184"""
        self._keys(lib().lcpp_radix_sort_keys_descending, "lcpp_radix_sort_keys_descending", temp_storage,
                   d_keys_in, d_keys_out, num_items, stream)

    def SortPairsDescending(self, temp_storage, d_keys_in, d_keys_out, d_values_in, d_values_out,
                            num_items: int, stream=None):
        """device_radix_sort.h:156-170 (stable: equal keys keep input order)"""
        self._pairs(lib().lcpp_radix_sort_pairs_descending, "lcpp_radix_sort_pairs_descending", temp_storage,
                    d_keys_in, d_keys_out, d_values_in, d_values_out, num_items, stream)


class DeviceSegmentReduce(_Module):
    """device/device_segment_reduce.h:26-349: Reduce / Sum / Min / Max / ArgMin / ArgMax over CSR
    begin/end offsets or over fixed-size segments (pass segment_size, an int, in place of the two
    offset buffers, as the reference's overloads do)."""


    @staticmethod
    def GetTempStorageBytes(dtype, num_item: int = 0) -> int:
        return _query(lib().lcpp_segment_reduce_temp_bytes, dtype_code(dtype), num_item)

    @staticmethod
    def GetArgTempStorageBytes(dtype, num_item: int, num_segments: int) -> int:
        """device_segment_reduce.h:77-89 (0 here: no key-value staging)"""
        return _query(lib().lcpp_segment_reduce_arg_temp_bytes, dtype_code(dtype), num_item, num_segments)

    # The library reads every segment the offsets name, as the reference does
    # (device_segment_reduce.h:353-381 validates nothing).  With
    # validate_offsets = True (or a debug stream) the CSR offsets are checked
    # against d_in on the host first, which synchronizes on a device-to-host
    # read; by default no call synchronizes.  Fixed-size segments are always
    # checked (host arithmetic only).
    validate_offsets = False

    def _check_ranges(self, d_in, num_segments, offsets):
        """Every segment must lie inside d_in: bad offsets raise instead of
        faulting the GPU."""
        if not num_segments:
            return
        if isinstance(offsets[0], int):
            size = offsets[0]
            if size < 0 or num_segments * size > d_in.numel():
                raise ValueError(f"{num_segments} segments of {size} exceed d_in ({d_in.numel()} elements)")
            if num_segments * size >= 1 << 32:
                raise ValueError("fixed-size segments must address fewer than 2^32 elements")
            return
        import torch

        d_begin_offsets, d_end_offsets = offsets
        _need(d_begin_offsets, num_segments, "d_begin_offsets")
        _need(d_end_offsets, num_segments, "d_end_offsets")
        if not (self.validate_offsets or self._debug):
            return
        b = d_begin_offsets[:num_segments].to(torch.int64)
        e = d_end_offsets[:num_segments].to(torch.int64)
        hi = torch.where(e > b, e, torch.zeros_like(e)).max().item()
        if hi > d_in.numel():
            raise ValueError(f"segment end {hi} exceeds d_in ({d_in.numel()} elements)")

    def _reduce(self, temp_storage, d_in, d_out, num_segments, offsets, op, init, stream, name):
        _need(d_out, num_segments, "d_out")
        _same_dtype(d_in, d_out, name)
        if op not in LCPP_OPS:
            raise ValueError(f"{name}: unsupported reduce_op {op!r}")
        self._check_ranges(d_in, num_segments, offsets)
        code = dtype_code(d_in.dtype)
        iv = _host_value(code, init) if init is not None else None
        ip = ctypes.c_void_p(iv.ctypes.data) if iv is not None else ctypes.c_void_p(0)
        L = lib()
        if isinstance(offsets[0], int):
            self._check(L.lcpp_segment_reduce_fixed(code, LCPP_OPS[op], _ptr(temp_storage), _nbytes(temp_storage),
                                              _ptr(d_in), _ptr(d_out), num_segments, offsets[0], ip, _stream(stream)),
                  "lcpp_segment_reduce_fixed", None, stream)
        else:
            self._check(L.lcpp_segment_reduce(code, LCPP_OPS[op], _ptr(temp_storage), _nbytes(temp_storage), _ptr(d_in),
                                        _ptr(d_out), num_segments, _ptr(offsets[0]), _ptr(offsets[1]), ip,
                                        _stream(stream)),
                  "lcpp_segment_reduce", None, stream)

    def Reduce(self, temp_storage, d_in, d_out, num_segments: int, *args, stream=None):
        """Reduce(temp, d_in, d_out, num_segments, d_begin_offsets, d_end_offsets, reduce_op, initial_value)
        or Reduce(temp, d_in, d_out, num_segments, segment_size, reduce_op, initial_value)
        (device_segment_reduce.h:94-123): d_out[s] = reduce_op(initial_value, fold of segment s).
        reduce_op: "sum" | "min" | "max"."""
        if isinstance(args[0], int):
            size, op, init = args
            offsets = (size,)
        else:
            b, e, op, init = args
            offsets = (b, e)
        self._reduce(temp_storage, d_in, d_out, num_segments, offsets, op, init, stream, "Reduce")

    @staticmethod
    def _offsets(args):
        return (args[0],) if isinstance(args[0], int) else (args[0], args[1])

    def Sum(self, temp_storage, d_in, d_out, num_segments: int, *offsets, stream=None):
        """device_segment_reduce.h:125-142 (CSR offsets, or a fixed segment_size)"""
        self._reduce(temp_storage, d_in, d_out, num_segments, self._offsets(offsets), "sum", None, stream, "Sum")

    def Min(self, temp_storage, d_in, d_out, num_segments: int, *offsets, stream=None):
        """device_segment_reduce.h:144-168 (init numeric max)"""
        self._reduce(temp_storage, d_in, d_out, num_segments, self._offsets(offsets), "min", None, stream, "Min")

    def Max(self, temp_storage, d_in, d_out, num_segments: int, *offsets, stream=None):
        """device_segment_reduce.h:170-195 (init numeric lowest)"""
        self._reduce(temp_storage, d_in, d_out, num_segments, self._offsets(offsets), "max", None, stream, "Max")

    def _arg(self, is_max, temp_storage, d_in, d_out, d_index_out, num_segments, offsets, stream):
        name = "ArgMax" if is_max else "ArgMin"
        _need(d_out, num_segments, "d_out")
        _need(d_index_out, num_segments, "d_index_out")
        _same_dtype(d_in, d_out, name)
        if d_index_out.element_size() != 4:
            raise TypeError(f"{name}: d_index_out must hold 32-bit indices")
        offsets = self._offsets(offsets)
        self._check_ranges(d_in, num_segments, offsets)
        L = lib()
        code = dtype_code(d_in.dtype)
        if isinstance(offsets[0], int):
            fn = L.lcpp_segment_reduce_argmax_fixed if is_max else L.lcpp_segment_reduce_argmin_fixed
            self._check(fn(code, _ptr(temp_storage), _nbytes(temp_storage), _ptr(d_in), _ptr(d_out), _ptr(d_index_out),
                     num_segments, offsets[0], _stream(stream)), fn.__name__, None, stream)
        else:
            fn = L.lcpp_segment_reduce_argmax if is_max else L.lcpp_segment_reduce_argmin
            self._check(fn(code, _ptr(temp_storage), _nbytes(temp_storage), _ptr(d_in), _ptr(d_out), _ptr(d_index_out),
                     num_segments, _ptr(offsets[0]), _ptr(offsets[1]), _stream(stream)), fn.__name__, None, stream)

    def ArgMax(self, temp_storage, d_in, d_out, d_index_out, num_segments: int, *offsets, stream=None):
        """device_segment_reduce.h:197-272: the largest value and its index within the segment
        (ties: the largest index); an empty segment gives (lowest, 1)."""
        self._arg(True, temp_storage, d_in, d_out, d_index_out, num_segments, offsets, stream)

    def ArgMin(self, temp_storage, d_in, d_out, d_index_out, num_segments: int, *offsets, stream=None):
        """device_segment_reduce.h:274-349: the smallest value and its index within the segment
        (ties: the smallest index); an empty segment gives (max, 1)."""
        self._arg(False, temp_storage, d_in, d_out, d_index_out, num_segments, offsets, stream)

    # the reference spells the CSR overload Argmin (device_segment_reduce.h:275)
    Argmin = ArgMin
