"""numpy binding of the CPU oracle (oracle/lcpp_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() (as
the checker) and bench.py's cpu_baseline leg.  The shipped library never
imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
lib_path = os.path.join(_DIR, "liblcpp_oracle.so")
_lib = None

I32, U32, F32, I64, U64, F64 = range(6)
OP_SUM, OP_MIN, OP_MAX = range(3)
_NP_CODE = {
    np.dtype(np.int32): I32,
    np.dtype(np.uint32): U32,
    np.dtype(np.float32): F32,
    np.dtype(np.int64): I64,
    np.dtype(np.uint64): U64,
    np.dtype(np.float64): F64,
}


def build() -> None:
    subprocess.run(["make", "-s", "-C", _DIR], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(lib_path):
            build()
        L = ctypes.CDLL(lib_path)
        vp, u64, i, u32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_uint32
        sig = {
            "lcor_splitmix64_next": (u64, [ctypes.POINTER(u64)]),
            "lcor_word": (u64, [u64, u64]),
            "lcor_gen_words": (None, [u64, u64, u64, vp]),
            "lcor_gen_reduce_i32": (None, [u64, u64, vp]),
            "lcor_gen_u8_u32": (None, [u64, u64, vp]),
            "lcor_gen_normal_f32": (None, [u64, u64, vp]),
            "lcor_gen_keys_u32": (None, [u64, u64, vp]),
            "lcor_gen_keys_u32_and3": (None, [u64, u64, u64, u64, vp]),
            "lcor_gen_keys_u64_low16": (None, [u64, u64, vp]),
            "lcor_gen_iota_u32": (None, [u64, vp]),
            "lcor_gen_segments": (i, [u64, u64, u64, u64, vp, vp]),
            "lcor_reduce": (i, [i, i, vp, u64, vp]),
            "lcor_reduce_f64": (i, [i, vp, u64, vp, vp]),
            "lcor_reduce_mt": (i, [i, i, vp, u64, vp, i]),
            "lcor_reduce_arg": (i, [i, i, vp, u64, vp, ctypes.POINTER(u32)]),
            "lcor_reduce_transform": (i, [i, i, i, vp, u64, vp, vp]),
            "lcor_scan": (i, [i, i, vp, vp, u64]),
            "lcor_scan_op": (i, [i, i, i, vp, vp, u64, vp]),
            "lcor_scan_f64": (i, [i, i, vp, vp, vp, u64]),
            "lcor_scan_mt": (i, [i, i, vp, vp, u64, i]),
            "lcor_lookback_kat": (i, [u32, i, vp, vp]),
            "lcor_lookback_bounded": (i, [vp, u32, i, u32, u32, u32, vp, vp, ctypes.POINTER(u32)]),
            "lcor_radix_sort": (i, [i, i, vp, vp, vp, vp, u64, i, i, u32]),
            "lcor_check_stable_pairs_u64_u32": (i, [vp, vp, vp, u64]),
            "lcor_check_sorted_permutation_u32": (i, [vp, vp, u64]),
            "lcor_scan_by_key": (i, [i, i, i, i, vp, vp, vp, u64, vp]),
            "lcor_scan_by_key_f64": (i, [i, i, i, vp, vp, vp, vp, u64]),
            "lcor_reduce_by_key": (i, [i, i, i, vp, vp, vp, vp, u64, ctypes.POINTER(u64)]),
            "lcor_reduce_by_key_f64": (i, [i, i, vp, vp, u64, vp, vp, ctypes.POINTER(u64)]),
            "lcor_segment_reduce": (i, [i, i, vp, vp, u64, vp, vp, vp]),
            "lcor_segment_reduce_arg": (i, [i, i, vp, vp, vp, u64, vp, vp]),
            "lcor_segment_reduce_f64": (i, [i, vp, u64, vp, vp, vp, vp]),
            "lcor_segment_reduce_mt": (i, [i, vp, vp, u64, vp, vp, i]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def _code(a: np.ndarray) -> int:
    return _NP_CODE[a.dtype]


def _ok(rc, what):
    if rc != 0:
        raise RuntimeError(f"oracle {what} failed ({rc})")


# ---------------------------------------------------------------- generators
def word(seed: int, i: int) -> int:
    return lib().lcor_word(seed, i)


def words(seed: int, n: int, start: int = 0) -> np.ndarray:
    out = np.empty(n, np.uint64)
    lib().lcor_gen_words(seed, start, n, _p(out))
    return out


def gen(kind: str, n: int, *seeds) -> np.ndarray:
    L = lib()
    if kind == "reduce_i32":
        out = np.empty(n, np.int32); L.lcor_gen_reduce_i32(seeds[0], n, _p(out))
    elif kind == "u8_u32":
        out = np.empty(n, np.uint32); L.lcor_gen_u8_u32(seeds[0], n, _p(out))
    elif kind == "normal_f32":
        out = np.empty(n, np.float32); L.lcor_gen_normal_f32(seeds[0], n, _p(out))
    elif kind == "keys_u32":
        out = np.empty(n, np.uint32); L.lcor_gen_keys_u32(seeds[0], n, _p(out))
    elif kind == "keys_u32_and3":
        out = np.empty(n, np.uint32); L.lcor_gen_keys_u32_and3(seeds[0], seeds[1], seeds[2], n, _p(out))
    elif kind == "keys_u64_low16":
        out = np.empty(n, np.uint64); L.lcor_gen_keys_u64_low16(seeds[0], n, _p(out))
    elif kind == "iota_u32":
        out = np.empty(n, np.uint32); L.lcor_gen_iota_u32(n, _p(out))
    else:
        raise ValueError(kind)
    return out


def segments(seed_empty: int, seed_len: int, n_items: int, n_segments: int):
    b = np.empty(n_segments, np.uint32)
    e = np.empty(n_segments, np.uint32)
    _ok(lib().lcor_gen_segments(seed_empty, seed_len, n_items, n_segments, _p(b), _p(e)), "gen_segments")
    return b, e


# ---------------------------------------------------------------- reduce
def reduce(op: int, a: np.ndarray, nthreads: int = 1):
    a = np.ascontiguousarray(a)
    out = np.zeros(1, a.dtype)
    if nthreads == 1:
        _ok(lib().lcor_reduce(op, _code(a), _p(a), a.size, _p(out)), "reduce")
    else:
        _ok(lib().lcor_reduce_mt(op, _code(a), _p(a), a.size, _p(out), nthreads), "reduce_mt")
    return out[0]


def reduce_arg(is_max: bool, a: np.ndarray):
    """(value, index) of ArgMax (is_max) / ArgMin."""
    a = np.ascontiguousarray(a)
    out = np.zeros(1, a.dtype)
    idx = ctypes.c_uint32()
    _ok(lib().lcor_reduce_arg(int(is_max), _code(a), _p(a), a.size, _p(out), ctypes.byref(idx)), "reduce_arg")
    return out[0], idx.value


XF_IDENTITY, XF_NEGATE, XF_ABS, XF_SQUARE = range(4)


def reduce_transform(op: int, xf: int, a: np.ndarray, init):
    a = np.ascontiguousarray(a)
    iv = np.array([init], dtype=a.dtype)
    out = np.zeros(1, a.dtype)
    _ok(lib().lcor_reduce_transform(op, xf, _code(a), _p(a), a.size, _p(iv), _p(out)), "reduce_transform")
    return out[0]


def reduce_f64(a: np.ndarray):
    """(double-precision sum, sum of |x|)."""
    a = np.ascontiguousarray(a)
    s = np.zeros(1, np.float64)
    ab = np.zeros(1, np.float64)
    _ok(lib().lcor_reduce_f64(_code(a), _p(a), a.size, _p(s), _p(ab)), "reduce_f64")
    return float(s[0]), float(ab[0])


# ---------------------------------------------------------------- scan
def scan(a: np.ndarray, inclusive: bool, nthreads: int = 1) -> np.ndarray:
    a = np.ascontiguousarray(a)
    out = np.empty_like(a)
    if nthreads == 1:
        _ok(lib().lcor_scan(int(inclusive), _code(a), _p(a), _p(out), a.size), "scan")
    else:
        _ok(lib().lcor_scan_mt(int(inclusive), _code(a), _p(a), _p(out), a.size, nthreads), "scan_mt")
    return out


def scan_op(a: np.ndarray, inclusive: bool, op: int, init=None) -> np.ndarray:
    """ExclusiveScan / InclusiveScan: a left fold from init (None = the op's identity)."""
    a = np.ascontiguousarray(a)
    out = np.empty_like(a)
    iv = np.array([init], dtype=a.dtype) if init is not None else None
    _ok(lib().lcor_scan_op(int(inclusive), op, _code(a), _p(a), _p(out), a.size, _p(iv) if iv is not None else None),
        "scan_op")
    return out


def scan_f64(a: np.ndarray, inclusive: bool):
    """(double-precision prefix sums, prefix sums of |x|)."""
    a = np.ascontiguousarray(a)
    out = np.empty(a.size, np.float64)
    ab = np.empty(a.size, np.float64)
    _ok(lib().lcor_scan_f64(int(inclusive), _code(a), _p(a), _p(out), _p(ab), a.size), "scan_f64")
    return out, ab


def lookback_kat(num_tiles: int, nthreads: int):
    ex = np.empty(num_tiles, np.int32)
    inc = np.empty(num_tiles, np.int32)
    _ok(lib().lcor_lookback_kat(num_tiles, nthreads, _p(ex), _p(inc)), "lookback_kat")
    return ex, inc


def lookback_bounded(agg: np.ndarray, nthreads: int, withhold: int = 0xFFFFFFFF, spin_limit: int = 1 << 20,
                     width: int = 16):
    """(exclusive, inclusive, status word) of the bounded look-back over the
    per-tile aggregates `agg` (int32, wrapping); tile `withhold` never publishes."""
    agg = np.ascontiguousarray(agg, dtype=np.int32)
    ex = np.empty(agg.size, np.int32)
    inc = np.empty(agg.size, np.int32)
    st = ctypes.c_uint32(0)
    _ok(lib().lcor_lookback_bounded(_p(agg), agg.size, nthreads, withhold, spin_limit, width, _p(ex), _p(inc),
                                    ctypes.byref(st)), "lookback_bounded")
    return ex, inc, st.value


# ---------------------------------------------------------------- sort
def radix_sort(keys: np.ndarray, values: np.ndarray | None = None, descending: bool = False, nthreads: int = 1,
               tile_items: int = 4096):
    keys = np.ascontiguousarray(keys)
    kout = np.empty_like(keys)
    vb = 0
    vout = None
    if values is not None:
        values = np.ascontiguousarray(values)
        vout = np.empty_like(values)
        vb = values.itemsize
    _ok(lib().lcor_radix_sort(_code(keys), vb, _p(keys), _p(kout),
                              _p(values) if values is not None else None,
                              _p(vout) if vout is not None else None,
                              keys.size, int(descending), nthreads, tile_items), "radix_sort")
    return (kout, vout) if values is not None else kout


def check_stable_pairs_u64_u32(keys_in, keys_out, vals_out) -> bool:
    return lib().lcor_check_stable_pairs_u64_u32(_p(keys_in), _p(keys_out), _p(vals_out), keys_in.size) == 1


def check_sorted_permutation_u32(keys_in, keys_out) -> bool:
    return lib().lcor_check_sorted_permutation_u32(_p(keys_in), _p(keys_out), keys_in.size) == 1


# ---------------------------------------------------------------- by key
def scan_by_key(keys: np.ndarray, values: np.ndarray, inclusive: bool, op: int = OP_SUM, init=0) -> np.ndarray:
    """ScanByKey over runs of equal consecutive keys (exclusive: init at heads)."""
    keys = np.ascontiguousarray(keys)
    values = np.ascontiguousarray(values)
    out = np.empty_like(values)
    iv = np.array([init], dtype=values.dtype)
    _ok(lib().lcor_scan_by_key(int(inclusive), op, _code(keys), _code(values), _p(keys), _p(values), _p(out),
                               values.size, _p(iv)), "scan_by_key")
    return out


def scan_by_key_f64(keys: np.ndarray, values: np.ndarray, inclusive: bool):
    """(double-precision segmented prefix sums, segmented prefix sums of |x|)."""
    keys = np.ascontiguousarray(keys)
    values = np.ascontiguousarray(values)
    out = np.empty(values.size, np.float64)
    ab = np.empty(values.size, np.float64)
    _ok(lib().lcor_scan_by_key_f64(int(inclusive), _code(keys), _code(values), _p(keys), _p(values), _p(out),
                                   _p(ab), values.size), "scan_by_key_f64")
    return out, ab


def reduce_by_key(keys: np.ndarray, values: np.ndarray, op: int = OP_SUM):
    """(unique keys, aggregates) of the runs of equal consecutive keys."""
    keys = np.ascontiguousarray(keys)
    values = np.ascontiguousarray(values)
    uk = np.empty_like(keys)
    ag = np.empty_like(values)
    runs = ctypes.c_uint64()
    _ok(lib().lcor_reduce_by_key(op, _code(keys), _code(values), _p(keys), _p(values), _p(uk), _p(ag), values.size,
                                 ctypes.byref(runs)), "reduce_by_key")
    return uk[: runs.value], ag[: runs.value]


def reduce_by_key_f64(keys: np.ndarray, values: np.ndarray):
    """(double-precision run sums, run sums of |x|)."""
    keys = np.ascontiguousarray(keys)
    values = np.ascontiguousarray(values)
    s = np.empty(max(values.size, 1), np.float64)
    ab = np.empty(max(values.size, 1), np.float64)
    runs = ctypes.c_uint64()
    _ok(lib().lcor_reduce_by_key_f64(_code(keys), _code(values), _p(keys), _p(values), values.size, _p(s), _p(ab),
                                     ctypes.byref(runs)), "reduce_by_key_f64")
    return s[: runs.value], ab[: runs.value]


# ---------------------------------------------------------------- segment reduce
def segment_reduce(op: int, a: np.ndarray, begin: np.ndarray, end: np.ndarray, init=None) -> np.ndarray:
    """out[s] = op(init, fold(a[begin[s]:end[s]])); init None = the op's identity."""
    a = np.ascontiguousarray(a)
    begin = np.ascontiguousarray(begin, np.uint32)
    end = np.ascontiguousarray(end, np.uint32)
    out = np.empty(begin.size, a.dtype)
    iv = np.array([init], dtype=a.dtype) if init is not None else None
    _ok(lib().lcor_segment_reduce(op, _code(a), _p(a), _p(out), begin.size, _p(begin), _p(end),
                                  _p(iv) if iv is not None else None), "segment_reduce")
    return out


def segment_reduce_arg(is_max: bool, a: np.ndarray, begin: np.ndarray, end: np.ndarray):
    """(values, relative indices) of ArgMax (is_max) / ArgMin per segment."""
    a = np.ascontiguousarray(a)
    begin = np.ascontiguousarray(begin, np.uint32)
    end = np.ascontiguousarray(end, np.uint32)
    out = np.empty(begin.size, a.dtype)
    idx = np.empty(begin.size, np.uint32)
    _ok(lib().lcor_segment_reduce_arg(int(is_max), _code(a), _p(a), _p(out), _p(idx), begin.size, _p(begin),
                                      _p(end)), "segment_reduce_arg")
    return out, idx


def fixed_segments(num_segments: int, segment_size: int):
    """CSR offsets of fixed-size segments: [s * size, (s + 1) * size)."""
    b = (np.arange(num_segments, dtype=np.uint64) * segment_size).astype(np.uint32)
    return b, (b.astype(np.uint64) + segment_size).astype(np.uint32)


def segment_reduce_f64(a: np.ndarray, begin: np.ndarray, end: np.ndarray):
    a = np.ascontiguousarray(a)
    s = np.empty(begin.size, np.float64)
    ab = np.empty(begin.size, np.float64)
    _ok(lib().lcor_segment_reduce_f64(_code(a), _p(a), begin.size, _p(begin), _p(end), _p(s), _p(ab)),
        "segment_reduce_f64")
    return s, ab


def segment_reduce_mt(a: np.ndarray, begin: np.ndarray, end: np.ndarray, nthreads: int) -> np.ndarray:
    out = np.empty(begin.size, a.dtype)
    _ok(lib().lcor_segment_reduce_mt(_code(a), _p(a), _p(out), begin.size, _p(begin), _p(end), nthreads),
        "segment_reduce_mt")
    return out
