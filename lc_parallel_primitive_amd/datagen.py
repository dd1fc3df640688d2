"""Seeded synthetic inputs of the benchmark configurations, generated in HBM.

Binding of liblcpp_datagen.so (csrc/datagen.hip).  Counter-based splitmix64:
element i of every stream can be regenerated on the host, so the GPU tests
can check full-size results without shipping inputs.
"""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
lib_path = os.path.join(_PKG, "liblcpp_datagen.so")
_lib = None

# fixed stream seeds of the benchmark configurations
SEED_REDUCE = 0xC1
SEED_SCAN_U32 = 0xC2A
SEED_SCAN_F32 = 0xC2B
SEED_SORT_U32 = 0xC3A
SEED_SORT_AND3 = (0xC3B1, 0xC3B2, 0xC3B3)
SEED_PAIRS_U64 = 0xC4
SEED_SEG_VALUES = 0xC5
SEED_SEG_EMPTY = 0xC5E
SEED_SEG_LEN = 0xC5F


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(lib_path):
            raise FileNotFoundError(f"{lib_path} is missing: build with `python lc_parallel_primitive_amd/build.py`")
        L = ctypes.CDLL(lib_path)
        u64, vp, i = ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int
        for name in ("lcpp_gen_reduce_i32", "lcpp_gen_u8_u32", "lcpp_gen_normal_f32", "lcpp_gen_keys_u32",
                     "lcpp_gen_keys_u64_low16", "lcpp_gen_keys_u64"):
            f = getattr(L, name)
            f.restype, f.argtypes = i, [u64, u64, vp, vp]
        L.lcpp_gen_keys_u32_and3.restype = i
        L.lcpp_gen_keys_u32_and3.argtypes = [u64, u64, u64, u64, vp, vp]
        L.lcpp_gen_iota_u32.restype = i
        L.lcpp_gen_iota_u32.argtypes = [u64, vp, vp]
        L.lcpp_copy_probe_u32.restype = i
        L.lcpp_copy_probe_u32.argtypes = [vp, vp, u64, vp]
        L.lcpp_dg_copy_shape.restype = i
        L.lcpp_dg_copy_shape.argtypes = [vp, vp, u64, ctypes.c_int, vp]
        L.lcpp_gen_segments_host.restype = i
        L.lcpp_gen_segments_host.argtypes = [u64, u64, u64, u64, vp, vp]
        L.lcpp_dg_sorted_hash_u32.restype = i
        L.lcpp_dg_sorted_hash_u32.argtypes = [vp, u64, vp, vp]
        L.lcpp_dg_check_stable_pairs_u32.restype = i
        L.lcpp_dg_check_stable_pairs_u32.argtypes = [vp, vp, vp, u64, vp, vp]
        L.lcpp_dg_lds_order_probe.restype = i
        L.lcpp_dg_lds_order_probe.argtypes = [u64, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, vp, vp]
        L.lcpp_dg_wave_kat.restype = i
        L.lcpp_dg_wave_kat.argtypes = [ctypes.c_int, vp, vp, vp, u64, vp]
        _lib = L
    return _lib


def _stream():
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _run(rc: int, what: str):
    if rc != 0:
        raise RuntimeError(f"{what} failed ({rc})")


def reduce_i32(n: int, seed: int = SEED_REDUCE, device="cuda"):
    """a_i = -1000 + floor(hi32(w_i) * 2001 / 2^32), uniform in [-1000, 1000]."""
    import torch

    t = torch.empty(n, dtype=torch.int32, device=device)
    _run(lib().lcpp_gen_reduce_i32(seed, n, t.data_ptr(), _stream()), "gen_reduce_i32")
    return t


def u8_u32(n: int, seed: int = SEED_SCAN_U32, device="cuda"):
    """x_i = hi32(w_i) >> 24, uniform in [0, 255]."""
    import torch

    t = torch.empty(n, dtype=torch.uint32, device=device)
    _run(lib().lcpp_gen_u8_u32(seed, n, t.data_ptr(), _stream()), "gen_u8_u32")
    return t


def normal_f32(n: int, seed: int = SEED_SCAN_F32, device="cuda"):
    """Box-Muller (cos branch) in double, cast to float32."""
    import torch

    t = torch.empty(n, dtype=torch.float32, device=device)
    _run(lib().lcpp_gen_normal_f32(seed, n, t.data_ptr(), _stream()), "gen_normal_f32")
    return t


def keys_u32(n: int, seed: int = SEED_SORT_U32, device="cuda"):
    """k_i = lo32(w_i): uniform over the full 32-bit range."""
    import torch

    t = torch.empty(n, dtype=torch.uint32, device=device)
    _run(lib().lcpp_gen_keys_u32(seed, n, t.data_ptr(), _stream()), "gen_keys_u32")
    return t


def keys_u32_and3(n: int, seeds=SEED_SORT_AND3, device="cuda"):
    """k_i = lo32(wA_i) & lo32(wB_i) & lo32(wC_i): each bit set with p = 1/8."""
    import torch

    t = torch.empty(n, dtype=torch.uint32, device=device)
    _run(lib().lcpp_gen_keys_u32_and3(seeds[0], seeds[1], seeds[2], n, t.data_ptr(), _stream()), "gen_and3")
    return t


def keys_u64_low16(n: int, seed: int = SEED_PAIRS_U64, device="cuda"):
    """k_i = w_i & 0xFFFF (upper 48 bits zero)."""
    import torch

    t = torch.empty(n, dtype=torch.uint64, device=device)
    _run(lib().lcpp_gen_keys_u64_low16(seed, n, t.data_ptr(), _stream()), "gen_keys_u64_low16")
    return t


SEED_PAIRS_U64_FULL = 0xC48


def keys_u64(n: int, seed: int = SEED_PAIRS_U64_FULL, device="cuda"):
    """k_i = w_i: uniform over the full 64-bit range (every onesweep pass moves data)."""
    import torch

    t = torch.empty(n, dtype=torch.uint64, device=device)
    _run(lib().lcpp_gen_keys_u64(seed, n, t.data_ptr(), _stream()), "gen_keys_u64")
    return t


SEED_BY_KEY = 0xB1


def run_keys_i32(n: int, log2_mean: int = 7, seed: int = SEED_BY_KEY, device="cuda"):
    """Keys made of runs of equal values with geometric lengths of mean
    2^log2_mean: key_i = #{j <= i : lo32(w_j) mod 2^log2_mean == 0}
    (int32; the host regenerates it from the same splitmix64 stream)."""
    import torch

    w = keys_u32(n, seed, device)
    heads = (w.view(torch.int32) & ((1 << log2_mean) - 1)) == 0
    del w
    return torch.cumsum(heads, dim=0, dtype=torch.int32)


def iota_u32(n: int, device="cuda"):
    import torch

    t = torch.empty(n, dtype=torch.uint32, device=device)
    _run(lib().lcpp_gen_iota_u32(n, t.data_ptr(), _stream()), "gen_iota_u32")
    return t


def segments(n_items: int, n_segments: int, seed_empty: int = SEED_SEG_EMPTY, seed_len: int = SEED_SEG_LEN):
    """CSR begin/end offsets (numpy uint32, host): 5 % empty, geometric lengths
    of mean 128/0.95 otherwise, rescaled to cover exactly n_items."""
    import numpy as np

    b = np.empty(n_segments, dtype=np.uint32)
    e = np.empty(n_segments, dtype=np.uint32)
    _run(lib().lcpp_gen_segments_host(seed_empty, seed_len, n_items, n_segments, b.ctypes.data, e.ctypes.data),
         "gen_segments_host")
    return b, e


def copy_probe(src, dst):
    """Streaming copy of a uint32 tensor (n % 4 == 0): calibration kernel for
    the HBM byte counters."""
    n = src.numel()
    _run(lib().lcpp_copy_probe_u32(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), n, _stream()),
         "copy_probe")


COPY_SHAPES = {
    0: "streaming copy, 16-byte vectors, 2 per thread",
    1: "scan tile: 256 thr x 20 x 16 B in registers, 4 WG/CU",
    2: "scan tile, copy's own occupancy",
    3: "grid-stride 16-byte copy, 2048 WGs",
    4: "onesweep tile: 512 thr x 32 dwords, sequential stores, 3 WG/CU",
    5: "onesweep tile -> 256 runs of 256 B, line-aligned, XCD runs of 16",
    6: "onesweep tile -> 256 runs, boundaries inside lines, XCD runs of 16",
    7: "onesweep tile -> 256 runs, boundaries inside lines, dispatch order",
    8: "onesweep tile -> 256 aligned runs, stores straddling lines",
}


def copy_shape(src, dst, shape):
    """Copy/permutation of a uint32 tensor in one of the access shapes of
    COPY_SHAPES (ceilings for the kernels that use those shapes)."""
    _run(lib().lcpp_dg_copy_shape(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), src.numel(), shape,
                                  _stream()), f"copy_shape {shape}")


def copy_shape_positions(n, shape):
    """numpy restatement of where shapes 4-8 write in[i] (host check of the
    probe's index arithmetic)."""
    import numpy as np

    tiles = n // 16384
    b = np.arange(tiles, dtype=np.int64)
    log_run = 0 if shape in (4, 7) else 4
    lg = log_run + 3
    g, r = b >> lg, b & ((1 << lg) - 1)
    full = ((g + 1) << lg) <= tiles
    tile_of_wg = np.where(full, (g << lg) + ((r & 7) << log_run) + (r >> 3), b)
    tid = np.arange(512, dtype=np.int64)
    lane, wave = tid & 63, tid >> 6
    u = np.arange(32, dtype=np.int64)
    region = n >> 8
    pos = np.empty(n, dtype=np.int64)
    for wg in range(tiles):
        t = int(tile_of_wg[wg])
        src = t * 16384 + wave[None, :] * 2048 + u[:, None] * 64 + lane[None, :]  # [u, tid]
        i = u[:, None] * 512 + tid[None, :]
        if shape == 4:
            p = t * 16384 + i
        elif shape == 5:
            p = (i >> 6) * region + t * 64 + (i & 63)
        elif shape == 8:
            i2 = (i + 16) & 16383
            p = (i2 >> 6) * region + t * 64 + (i2 & 63)
        else:
            kk, rr = i >> 7, i & 127
            a = (kk * 37) % 29 + 1
            odd = t & 1
            split = 64 - a if odd else 64 + a
            d = np.where(rr < split, 2 * kk, 2 * kk + 1)
            within = np.where(rr < split, rr, rr - split)
            pre = t * 64 + (np.where(d & 1, -a, a) if odd else 0)
            p = d * region + pre + within
        pos[src.ravel()] = p.ravel()
    return pos


# ---------------------------------------------------------------- device-side checkers (tests)
def sorted_hash_u32(t):
    """(descents, sum mod 2^64, sum of mix64 mod 2^64) of a uint32 device
    tensor: descents == 0 means sorted; the sums are equal for equal multisets."""
    import torch

    out = torch.zeros(3, dtype=torch.uint64, device=t.device)
    _run(lib().lcpp_dg_sorted_hash_u32(ctypes.c_void_p(t.data_ptr()), t.numel(), ctypes.c_void_p(out.data_ptr()),
                                       _stream()), "sorted_hash_u32")
    h = out.cpu().view(torch.int64).tolist()
    return tuple(x & 0xFFFFFFFFFFFFFFFF for x in h)


def check_stable_pairs_u32(keys_in, keys_out, vals_out) -> int:
    """Bad positions of a stable uint32/uint32 sort whose values were the input
    indices (0 <=> keys_out/vals_out is exactly the stable sort)."""
    import torch

    bad = torch.zeros(1, dtype=torch.uint64, device=keys_in.device)
    _run(lib().lcpp_dg_check_stable_pairs_u32(ctypes.c_void_p(keys_in.data_ptr()), ctypes.c_void_p(keys_out.data_ptr()),
                                              ctypes.c_void_p(vals_out.data_ptr()), keys_in.numel(),
                                              ctypes.c_void_p(bad.data_ptr()), _stream()), "check_stable_pairs_u32")
    return int(bad.cpu().view(torch.int64).item())


def lds_order_probe(seed: int, pattern: int, waves: int, rounds: int) -> int:
    """Lanes whose returning LDS atomic add broke lane order (see datagen.hip)."""
    import torch

    v = torch.zeros(1, dtype=torch.uint64, device="cuda")
    _run(lib().lcpp_dg_lds_order_probe(seed, pattern, waves, rounds, ctypes.c_void_p(v.data_ptr()), _stream()),
         "lds_order_probe")
    return int(v.cpu().view(torch.int64).item())


WAVE_KAT_KINDS = {"reduce_sum": 0, "exclusive_sum": 1, "inclusive_sum": 2, "segmented_sum": 3, "flag_rank": 4,
                  "inclusive_max": 5, "reduce_min": 6, "shift_up": 7}


def wave_kat(kind: str, x, flags=None):
    """One of the wave64 primitive cases of datagen.hip's wave_kat_kernel over
    int32 device tensor x (length a multiple of 64); returns the device output
    (one value per wave for the reductions, one per element otherwise)."""
    import torch

    k = WAVE_KAT_KINDS[kind]
    n = x.numel()
    out = torch.empty(n // 64 if k in (0, 6) else n, dtype=torch.int32, device=x.device)
    fp = ctypes.c_void_p(flags.data_ptr()) if flags is not None else None
    _run(lib().lcpp_dg_wave_kat(k, ctypes.c_void_p(x.data_ptr()), fp, ctypes.c_void_p(out.data_ptr()), n,
                                _stream()), f"wave_kat {kind}")
    return out
