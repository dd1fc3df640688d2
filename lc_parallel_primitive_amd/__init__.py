"""MI355X-native (gfx950) device-level parallel primitives.

Python mirror of LCPP's host API (src/lcpp/device/device_*.h of
Ligo04/lc_parallel_primitive) over the C ABI in include/lcpp_amd.h.  Device
memory is held in torch tensors (plumbing only); every call goes through
the hand-written HIP kernels of liblcpp_amd.so and fails loudly when that
library is missing.

    from lc_parallel_primitive_amd import DeviceReduce
    temp = torch.empty(DeviceReduce.GetTempStorageBytes(torch.int32, n), dtype=torch.uint8, device="cuda")
    DeviceReduce().Sum(temp, d_in, d_out, n)
"""
from __future__ import annotations

import ctypes
import os

from ._capi import (  # noqa: F401
    LCPP_DTYPES,
    LcppError,
    dtype_code,
    lib,
    lib_path,
    profile_disable,
    profile_enable,
    profile_read,
)
from .device import DeviceRadixSort, DeviceReduce, DeviceScan, DeviceSegmentReduce  # noqa: F401

__all__ = [
    "DeviceReduce",
    "DeviceScan",
    "DeviceRadixSort",
    "DeviceSegmentReduce",
    "LcppError",
    "lib",
    "lib_path",
    "dtype_code",
    "profile_enable",
    "profile_disable",
    "profile_read",
]

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
