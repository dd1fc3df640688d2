"""ctypes binding of include/lcpp_amd.h (liblcpp_amd.so)."""
from __future__ import annotations

import ctypes
import os
import threading

_PKG = os.path.dirname(os.path.abspath(__file__))
lib_path = os.path.join(_PKG, "liblcpp_amd.so")

LCPP_INT32, LCPP_UINT32, LCPP_FLOAT32, LCPP_INT64, LCPP_UINT64, LCPP_FLOAT64 = range(6)
LCPP_OPS = {"sum": 0, "min": 1, "max": 2}
LCPP_TRANSFORMS = {"identity": 0, "negate": 1, "abs": 2, "square": 3}
LCPP_DTYPES = {
    "int32": LCPP_INT32,
    "uint32": LCPP_UINT32,
    "float32": LCPP_FLOAT32,
    "int64": LCPP_INT64,
    "uint64": LCPP_UINT64,
    "float64": LCPP_FLOAT64,
}

# name -> (restype, argtypes)
_c_size_p = ctypes.POINTER(ctypes.c_size_t)
_vp = ctypes.c_void_p
_u64 = ctypes.c_uint64
_i = ctypes.c_int
SIGNATURES = {
    "lcpp_version": (_i, []),
    "lcpp_status_string": (ctypes.c_char_p, [_i]),
    "lcpp_reduce_temp_bytes": (_i, [_i, _u64, _c_size_p]),
    "lcpp_reduce_sum": (_i, [_i, _vp, ctypes.c_size_t, _vp, _vp, _u64, _vp]),
    "lcpp_reduce_min": (_i, [_i, _vp, ctypes.c_size_t, _vp, _vp, _u64, _vp]),
    "lcpp_reduce_max": (_i, [_i, _vp, ctypes.c_size_t, _vp, _vp, _u64, _vp]),
    "lcpp_reduce_transform": (_i, [_i, _i, _i, _vp, ctypes.c_size_t, _vp, _vp, _u64, _vp, _vp]),
    "lcpp_reduce_arg_temp_bytes": (_i, [_i, _u64, _c_size_p]),
    "lcpp_reduce_argmin": (_i, [_i, _vp, ctypes.c_size_t, _vp, _vp, _vp, _u64, _vp]),
    "lcpp_reduce_argmax": (_i, [_i, _vp, ctypes.c_size_t, _vp, _vp, _vp, _u64, _vp]),
    "lcpp_scan_temp_bytes": (_i, [_i, _u64, _c_size_p]),
    "lcpp_scan_exclusive_sum": (_i, [_i, _vp, ctypes.c_size_t, _vp, _vp, _u64, _vp]),
    "lcpp_scan_inclusive_sum": (_i, [_i, _vp, ctypes.c_size_t, _vp, _vp, _u64, _vp]),
    "lcpp_scan_exclusive": (_i, [_i, _i, _vp, ctypes.c_size_t, _vp, _vp, _u64, _vp, _vp]),
    "lcpp_scan_inclusive": (_i, [_i, _i, _vp, ctypes.c_size_t, _vp, _vp, _u64, _vp, _vp]),
    "lcpp_scan_exclusive_sum_noalloc": (_i, [_i, _vp, _vp, _u64, _vp]),
    "lcpp_radix_sort_keys_temp_bytes": (_i, [_i, _u64, _c_size_p]),
    "lcpp_radix_sort_keys": (_i, [_i, _vp, ctypes.c_size_t, _vp, _vp, _u64, _vp]),
    "lcpp_radix_sort_pairs_temp_bytes": (_i, [_i, _i, _u64, _c_size_p]),
    "lcpp_radix_sort_pairs": (_i, [_i, _i, _vp, ctypes.c_size_t, _vp, _vp, _vp, _vp, _u64, _vp]),
    "lcpp_radix_sort_keys_descending": (_i, [_i, _vp, ctypes.c_size_t, _vp, _vp, _u64, _vp]),
    "lcpp_radix_sort_pairs_descending": (_i, [_i, _i, _vp, ctypes.c_size_t, _vp, _vp, _vp, _vp, _u64, _vp]),
    "lcpp_radix_sort_rank_path": (_i, [ctypes.POINTER(_i)]),
    "lcpp_test_set_sort_rank_path": (_i, [_i]),
    "lcpp_scan_by_key_temp_bytes": (_i, [_i, _i, _u64, _c_size_p]),
    "lcpp_scan_exclusive_by_key": (_i, [_i, _i, _i, _vp, ctypes.c_size_t, _vp, _vp, _vp, _u64, _vp, _vp]),
    "lcpp_scan_inclusive_by_key": (_i, [_i, _i, _i, _vp, ctypes.c_size_t, _vp, _vp, _vp, _u64, _vp, _vp]),
    "lcpp_scan_exclusive_sum_by_key": (_i, [_i, _i, _vp, ctypes.c_size_t, _vp, _vp, _vp, _u64, _vp]),
    "lcpp_scan_inclusive_sum_by_key": (_i, [_i, _i, _vp, ctypes.c_size_t, _vp, _vp, _vp, _u64, _vp]),
    "lcpp_reduce_by_key_temp_bytes": (_i, [_i, _i, _u64, _c_size_p]),
    "lcpp_reduce_by_key": (_i, [_i, _i, _i, _vp, ctypes.c_size_t, _vp, _vp, _vp, _vp, _vp, _u64, _vp]),
    "lcpp_segment_reduce_temp_bytes": (_i, [_i, _u64, _c_size_p]),
    "lcpp_segment_reduce_sum": (_i, [_i, _vp, ctypes.c_size_t, _vp, _vp, _u64, _vp, _vp, _vp]),
    "lcpp_segment_reduce": (_i, [_i, _i, _vp, ctypes.c_size_t, _vp, _vp, _u64, _vp, _vp, _vp, _vp]),
    "lcpp_segment_reduce_fixed": (_i, [_i, _i, _vp, ctypes.c_size_t, _vp, _vp, _u64, ctypes.c_uint32, _vp, _vp]),
    "lcpp_segment_reduce_arg_temp_bytes": (_i, [_i, _u64, _u64, _c_size_p]),
    "lcpp_segment_reduce_argmin": (_i, [_i, _vp, ctypes.c_size_t, _vp, _vp, _vp, _u64, _vp, _vp, _vp]),
    "lcpp_segment_reduce_argmax": (_i, [_i, _vp, ctypes.c_size_t, _vp, _vp, _vp, _u64, _vp, _vp, _vp]),
    "lcpp_segment_reduce_argmin_fixed": (_i, [_i, _vp, ctypes.c_size_t, _vp, _vp, _vp, _u64, ctypes.c_uint32, _vp]),
    "lcpp_segment_reduce_argmax_fixed": (_i, [_i, _vp, ctypes.c_size_t, _vp, _vp, _vp, _u64, ctypes.c_uint32, _vp]),
    "lcpp_temp_status": (_i, [_vp, ctypes.c_size_t, _vp]),
    "lcpp_temp_status_record": (_i, [_vp, ctypes.c_size_t, _vp, _vp]),
    "lcpp_device_status_decode": (_i, [ctypes.c_uint32]),
    "lcpp_stream_sync": (_i, [_vp]),
    "lcpp_test_set_lookback_fault": (_i, [ctypes.c_uint32, ctypes.c_uint32]),
    "lcpp_profile_enable": (_i, [_i]),
    "lcpp_profile_count": (_i, []),
    "lcpp_profile_get": (_i, [_i, ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(_u64), ctypes.POINTER(ctypes.c_double)]),
}

_lock = threading.Lock()
_lib = None


class LcppError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        name = lib().lcpp_status_string(status).decode() if _lib is not None else str(status)
        super().__init__(f"{what} failed: {name} ({status})")


def lib() -> ctypes.CDLL:
    """Load liblcpp_amd.so (built by lc_parallel_primitive_amd/build.py).

    Raises FileNotFoundError when the library has not been built: there is
    no fallback implementation."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(lib_path):
                raise FileNotFoundError(
                    f"{lib_path} is missing: build it with `python lc_parallel_primitive_amd/build.py`"
                )
            L = ctypes.CDLL(lib_path)
            for name, (res, args) in SIGNATURES.items():
                f = getattr(L, name)
                f.restype = res
                f.argtypes = args
            _lib = L
        return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        raise LcppError(status, what)


def dtype_code(dtype) -> int:
    """lcpp_dtype of a torch / numpy dtype or a dtype name."""
    name = str(dtype).replace("torch.", "").replace("numpy.", "")
    if name not in LCPP_DTYPES:
        raise TypeError(f"unsupported dtype {dtype}")
    return LCPP_DTYPES[name]


def profile_enable() -> None:
    check(lib().lcpp_profile_enable(1), "lcpp_profile_enable")


def profile_disable() -> None:
    check(lib().lcpp_profile_enable(0), "lcpp_profile_enable")


def profile_read() -> dict:
    """{kernel name: (launches, total ms)} of the launches since profile_enable()."""
    L = lib()
    n = L.lcpp_profile_count()
    if n < 0:
        raise LcppError(n, "lcpp_profile_count")
    out = {}
    buf = ctypes.create_string_buffer(128)
    for i in range(n):
        launches = _u64()
        ms = ctypes.c_double()
        check(L.lcpp_profile_get(i, buf, 128, ctypes.byref(launches), ctypes.byref(ms)), "lcpp_profile_get")
        out[buf.value.decode()] = (launches.value, ms.value)
    return out
