"""Regenerate the golden fixtures of tests/golden/.

Compiles make_golden.cpp with g++ (libstdc++: std::mt19937, std::shuffle and
std::uniform_real_distribution as the reference's tests call them) and
writes the raw arrays listed in golden.json next to this script.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))

MANIFEST = {
    "generator": "make_golden.cpp (g++ / libstdc++, std::mt19937(114521))",
    "files": {
        "reduce_shuffled_4096_i32.bin": ["int32", "device_reduce_test.cpp:53-62 input (0..4095 shuffled)"],
        "reduce_shuffled_4096_expect_min_max_sum_i32.bin": ["int32", "std::min_element, max_element, accumulate"],
        "segment_shuffled_1024_i32.bin": ["int32", "device_segment_reduce.cpp:64-72 input"],
        "segment_shuffled_1024_begin_u32.bin": ["uint32", "device_segment_reduce.cpp:78-85 begin offsets"],
        "segment_shuffled_1024_end_u32.bin": ["uint32", "device_segment_reduce.cpp:78-85 end offsets"],
        "segment_shuffled_1024_expect_i32.bin": ["int32", "std::accumulate per segment"],
        "sort_pairs_16384_keys_in_u32.bin": ["uint32", "device_radix_sort_one_sweep.cpp:155-175 keys, n=16384"],
        "sort_pairs_16384_vals_in_f32.bin": ["float32", "device_radix_sort_one_sweep.cpp:155-175 values"],
        "sort_pairs_16384_keys_expect_u32.bin": ["uint32", "std::sort by key"],
        "sort_pairs_16384_vals_expect_f32.bin": ["float32", "values in key order"],
        "sort_pairs_desc_16384_keys_in_u32.bin": ["uint32", "device_radix_sort_one_sweep.cpp:155-175 second keys, n=16384"],
        "sort_pairs_desc_16384_vals_in_f32.bin": ["float32", "device_radix_sort_one_sweep.cpp:155-175 second values"],
        "sort_pairs_desc_16384_keys_expect_u32.bin": ["uint32", "std::sort by key, greater"],
        "sort_pairs_desc_16384_vals_expect_f32.bin": ["float32", "values in descending key order"],
    },
}
for n in (32, 256, 4096):
    for d in ("asc", "desc"):
        MANIFEST["files"][f"sort_float_{n}_{d}_in_f32.bin"] = [
            "float32", f"device_radix_sort_one_sweep.cpp:65-76 {d} keys, n={n}"]
        MANIFEST["files"][f"sort_float_{n}_{d}_expect_f32.bin"] = [
            "float32", f"std::sort ({'less' if d == 'asc' else 'greater'})"]


def main() -> None:
    with tempfile.TemporaryDirectory() as td:
        exe = os.path.join(td, "make_golden")
        subprocess.run(["g++", "-O2", "-std=c++17", os.path.join(HERE, "make_golden.cpp"), "-o", exe], check=True)
        subprocess.run([exe, HERE], check=True)
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(MANIFEST, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
