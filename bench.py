#!/usr/bin/env python3
"""Benchmark of the MI355X-native LCPP device primitives (one GPU).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-secondary] [--no-cpu-baseline]

Headline (BASELINE.json metric): DeviceRadixSort::SortKeys on 2^28 uint32
keys uniform over the full 32-bit range (histogram + 4 onesweep passes),
keys resident in HBM.  One step = one SortKeys call through the C ABI.
Prints ONE JSON line.  `roofline` is the dominant kernel (the onesweep pass)
measured live with HIP events recorded by the library on the launch stream;
`secondary` holds the scan / reduce / pairs / low-entropy / segment-reduce
configurations; `cpu_baseline` times the CPU onesweep restatement (oracle/)
on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "rs_onesweep_u32_2p28_hbm_bytes.txt")


def measured_traffic():
    """HBM bytes per onesweep launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE runs (copy-calibrated), or None when that summary is absent."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if "traffic_bytes_per_launch" in line:
                    return int(line.split("=")[1].split()[0])
    except (OSError, ValueError, IndexError):
        pass
    return None


def progress(msg):
    """One line per finished stage on stderr (the JSON line stays alone on stdout)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default=None, help="run one secondary workload by name (profiling)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 2^28 x uint32 streaming copy (calibrates rocprofv3 byte counters)")
    return ap.parse_args()


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only: every box has a single MI355X; "
                                   "run with --gpus 1 (the multi-GPU sharding is described in DESIGN.md)"}))
        sys.exit(2)

    import torch

    import lc_parallel_primitive_amd as lcpp
    from lc_parallel_primitive_amd import datagen

    L = lcpp.lib()
    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)

    def tmp_bytes(fn, *a):
        b = ctypes.c_size_t()
        lcpp._capi.check(fn(*a, ctypes.byref(b)), fn.__name__)
        return b.value

    def timed(call, steps, warmup):
        for _ in range(warmup):
            call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            call()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps  # ms per step

    def kernel_ms(call, steps, name):
        """Average device duration of kernel `name` over `steps` calls (HIP events
        recorded by the library around each launch, on the launch stream)."""
        lcpp.profile_enable()
        for _ in range(steps):
            call()
        torch.cuda.synchronize()
        rec = lcpp.profile_read()
        lcpp.profile_disable()
        launches, total = rec[name]
        return total / launches, launches, rec

    U32, F32, I32, U64 = 1, 2, 0, 4
    chk = lcpp._capi.check

    if args.copy_probe:
        n = 1 << 28
        src = datagen.keys_u32(n)
        dst = torch.empty_like(src)
        ms = timed(lambda: datagen.copy_probe(src, dst), args.steps, args.warmup)
        print(json.dumps({"copy_probe": {"bytes_read_per_launch": 4 * n, "bytes_written_per_launch": 4 * n,
                                         "launches": args.steps + args.warmup, "ms": round(ms, 4),
                                         "GB/s": round(8 * n / (ms * 1e-3) / 1e9, 1)}}), flush=True)
        return

    # ------------------------------------------------------------ headline: SortKeys u32 2^28
    n = 1 << 28
    keys = datagen.keys_u32(n)
    out = torch.empty_like(keys)
    tb = tmp_bytes(L.lcpp_radix_sort_keys_temp_bytes, U32, n)
    temp = torch.empty(tb, dtype=torch.uint8, device="cuda")

    def sort_call():
        chk(L.lcpp_radix_sort_keys(U32, ctypes.c_void_p(temp.data_ptr()), tb, ctypes.c_void_p(keys.data_ptr()),
                                   ctypes.c_void_p(out.data_ptr()), n, sp), "sort")

    ms = timed(sort_call, args.steps, args.warmup)
    gkeys = n / (ms * 1e-3) / 1e9
    progress(f"SortKeys u32 2^28: {ms:.4f} ms/step, {gkeys:.2f} Gkeys/s")
    pass_ms, pass_launches, rec = kernel_ms(sort_call, max(2, args.steps // 4), "rs_onesweep")
    pass_bytes = 8 * n  # read 4N + write 4N per onesweep pass (algorithmic)
    achieved = pass_bytes / (pass_ms * 1e-3) / 1e9
    breakdown = {k: round(v[1] / v[0] * 1e3, 2) for k, v in rec.items()}  # us per launch
    del temp, out

    result = {
        "metric": "SortKeys u32 2^28 Gkeys/s",
        "value": round(gkeys, 3),
        "unit": "Gkeys/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic (splitmix64 keys generated in HBM, seed 0xC3A)",
        "config": {
            "workload": "DeviceRadixSort::SortKeys uint32 N=2^28 uniform full 32-bit range (BASELINE configs[2])",
            "n": n,
            "passes": 4,
            "algorithmic_bytes_per_sort": 36 * n,
            "sort_roofline_frac": round(36 * n / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "us_per_launch": breakdown,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "rs_onesweep (one 8-bit digit pass)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "traffic_source": "rocprofv3 FETCH_SIZE+WRITE_SIZE, copy-calibrated: profiles/rs_onesweep_u32_2p28_hbm_bytes.txt",
            "bytes_per_launch": pass_bytes,
            "avg_launch_us": round(pass_ms * 1e3, 2),
            "launches": pass_launches,
        },
    }

    # ------------------------------------------------------------ secondary configurations
    if not args.no_secondary:
        sec = []

        def add(name, unit_bytes, call, steps, kname, items=None, unit="GB/s"):
            t = timed(call, steps, 2)
            kms, _, _ = kernel_ms(call, max(2, steps // 2), kname)
            gbs = unit_bytes / (t * 1e-3) / 1e9
            entry = {"workload": name, "ms": round(t, 4), "GB/s": round(gbs, 1),
                     "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                     "dominant_kernel": kname, "kernel_us": round(kms * 1e3, 2)}
            if items is not None:
                entry["Gitems/s"] = round(items / (t * 1e-3) / 1e9, 3)
            sec.append(entry)
            progress(f"{name}: {entry['ms']} ms")

        def want(name):
            return args.only is None or args.only == name

        if want("reduce"):
            n = 1 << 28
            x = datagen.reduce_i32(n)
            o1 = torch.empty(1, dtype=torch.int32, device="cuda")
            tb = tmp_bytes(L.lcpp_reduce_temp_bytes, I32, n)
            t1 = torch.empty(max(tb, 1), dtype=torch.uint8, device="cuda")
            add("DeviceReduce::Sum int32 N=2^28", 4 * n + 4,
                lambda: chk(L.lcpp_reduce_sum(I32, ctypes.c_void_p(t1.data_ptr()), tb, ctypes.c_void_p(x.data_ptr()),
                                              ctypes.c_void_p(o1.data_ptr()), n, sp), "reduce"), 20, "reduce_partials")
            n24 = 1 << 24
            add("DeviceReduce::Sum int32 N=2^24 (configs[0])", 4 * n24 + 4,
                lambda: chk(L.lcpp_reduce_sum(I32, ctypes.c_void_p(t1.data_ptr()), tb, ctypes.c_void_p(x.data_ptr()),
                                              ctypes.c_void_p(o1.data_ptr()), n24, sp), "reduce"), 50, "reduce_partials")
            ta = tmp_bytes(L.lcpp_reduce_arg_temp_bytes, I32, n)
            t2 = torch.empty(max(ta, 1), dtype=torch.uint8, device="cuda")
            ix = torch.empty(1, dtype=torch.int32, device="cuda")
            add("DeviceReduce::ArgMin int32 N=2^28", 4 * n + 8,
                lambda: chk(L.lcpp_reduce_argmin(I32, ctypes.c_void_p(t2.data_ptr()), ta,
                                                 ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(o1.data_ptr()),
                                                 ctypes.c_void_p(ix.data_ptr()), n, sp), "argmin"), 20, "arg_partials")
            del x, t1, t2
        if want("scan"):
            n = 1 << 28
            x = datagen.u8_u32(n)
            y = torch.empty_like(x)
            tb = tmp_bytes(L.lcpp_scan_temp_bytes, U32, n)
            t1 = torch.empty(tb, dtype=torch.uint8, device="cuda")
            add("DeviceScan::ExclusiveSum uint32 N=2^28", 8 * n,
                lambda: chk(L.lcpp_scan_exclusive_sum(U32, ctypes.c_void_p(t1.data_ptr()), tb,
                                                      ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()),
                                                      n, sp), "scan"), 20, "scan_exclusive")
            del x
            xf = datagen.normal_f32(n)
            yf = torch.empty_like(xf)
            add("DeviceScan::InclusiveSum float32 N=2^28", 8 * n,
                lambda: chk(L.lcpp_scan_inclusive_sum(F32, ctypes.c_void_p(t1.data_ptr()), tb,
                                                      ctypes.c_void_p(xf.data_ptr()), ctypes.c_void_p(yf.data_ptr()),
                                                      n, sp), "scan"), 20, "scan_inclusive")
            del xf, yf, y, t1
        if want("sort_and3"):
            n = 1 << 28
            k = datagen.keys_u32_and3(n)
            ko = torch.empty_like(k)
            tb = tmp_bytes(L.lcpp_radix_sort_keys_temp_bytes, U32, n)
            t1 = torch.empty(tb, dtype=torch.uint8, device="cuda")
            add("DeviceRadixSort::SortKeys uint32 N=2^28 AND-of-3 (low entropy)", 36 * n,
                lambda: chk(L.lcpp_radix_sort_keys(U32, ctypes.c_void_p(t1.data_ptr()), tb,
                                                   ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(ko.data_ptr()), n,
                                                   sp), "sort"), 10, "rs_onesweep", items=n)
            del k, ko, t1
        if want("pairs"):
            n = 1 << 27
            k = datagen.keys_u64_low16(n)
            v = datagen.iota_u32(n)
            ko, vo = torch.empty_like(k), torch.empty_like(v)
            tb = tmp_bytes(L.lcpp_radix_sort_pairs_temp_bytes, U64, U32, n)
            t1 = torch.empty(tb, dtype=torch.uint8, device="cuda")
            # 16 random low bits: passes 2..7 see one digit for every key and are
            # skipped (identity permutations), so the bytes counted are the
            # histogram (8 B) plus the two passes that move data (2 x 24 B); the
            # reference's eight passes would move 200 B per pair
            add("DeviceRadixSort::SortPairs uint64->uint32 N=2^27 (16 random low bits; 2 of 8 digit passes move data)",
                56 * n,
                lambda: chk(L.lcpp_radix_sort_pairs(U64, U32, ctypes.c_void_p(t1.data_ptr()), tb,
                                                    ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(ko.data_ptr()),
                                                    ctypes.c_void_p(v.data_ptr()), ctypes.c_void_p(vo.data_ptr()),
                                                    n, sp), "pairs"), 5, "rs_onesweep", items=n)
            del k, v, ko, vo, t1
        if want("by_key"):
            n = 1 << 28
            k = datagen.run_keys_i32(n, 7)
            runs = int(k[-1].item()) - int(k[0].item()) + 1
            x = datagen.normal_f32(n, seed=datagen.SEED_SEG_VALUES)
            y = torch.empty_like(x)
            tb = tmp_bytes(L.lcpp_scan_by_key_temp_bytes, I32, F32, n)
            t1 = torch.empty(tb, dtype=torch.uint8, device="cuda")
            add("DeviceScan::InclusiveSumByKey int32 keys (runs of mean 128) -> float32 N=2^28", 12 * n,
                lambda: chk(L.lcpp_scan_inclusive_sum_by_key(I32, F32, ctypes.c_void_p(t1.data_ptr()), tb,
                                                             ctypes.c_void_p(k.data_ptr()),
                                                             ctypes.c_void_p(x.data_ptr()),
                                                             ctypes.c_void_p(y.data_ptr()), n, sp), "sbk"),
                20, "scan_by_key_inclusive")
            del y, t1
            uk = torch.empty_like(k)
            ag = torch.empty_like(x)
            nr = torch.zeros(1, dtype=torch.int32, device="cuda")
            tb = tmp_bytes(L.lcpp_reduce_by_key_temp_bytes, I32, F32, n)
            t1 = torch.empty(tb, dtype=torch.uint8, device="cuda")
            add("DeviceReduce::ReduceByKey sum int32 keys (runs of mean 128) -> float32 N=2^28", 8 * n + 8 * runs,
                lambda: chk(L.lcpp_reduce_by_key(I32, F32, 0, ctypes.c_void_p(t1.data_ptr()), tb,
                                                 ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                                 ctypes.c_void_p(uk.data_ptr()), ctypes.c_void_p(ag.data_ptr()),
                                                 ctypes.c_void_p(nr.data_ptr()), n, sp), "rbk"),
                20, "reduce_by_key")
            del k, x, uk, ag, t1
        if want("segment"):
            n, S = 1 << 27, 1 << 20
            x = datagen.normal_f32(n, seed=datagen.SEED_SEG_VALUES)
            b, e = datagen.segments(n, S)
            db = torch.from_numpy(b).cuda()
            de = torch.from_numpy(e).cuda()
            y = torch.empty(S, dtype=torch.float32, device="cuda")
            add("DeviceSegmentReduce::Sum float32 N=2^27 S=2^20", 4 * n + 12 * S,
                lambda: chk(L.lcpp_segment_reduce_sum(F32, None, 0, ctypes.c_void_p(x.data_ptr()),
                                                      ctypes.c_void_p(y.data_ptr()), S, ctypes.c_void_p(db.data_ptr()),
                                                      ctypes.c_void_p(de.data_ptr()), sp), "segment"), 20,
                "segment_reduce")
            del x, y, db, de
        result["secondary"] = sec

    # ------------------------------------------------------------ CPU baseline (oracle onesweep port)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
        progress(f"cpu baseline: {result['cpu_baseline']['value']} Gkeys/s")

    print(json.dumps(result), flush=True)


def cpu_baseline():
    import numpy as np

    from oracle import oracle as o

    cores = len(os.sched_getaffinity(0))
    threads = max(1, min(cores, 16))  # the GPU box's CPU share is 16 threads
    n = 1 << 25
    keys = o.gen("keys_u32", n, 0xC3A)
    o.radix_sort(keys[: 1 << 20], nthreads=threads)  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        o.radix_sort(keys, nthreads=threads)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(n / med / 1e9, 4),
        "unit": "Gkeys/s",
        "cores": threads,
        "kind": "port",
        "sample": f"SortKeys uint32 N=2^25 uniform (same generator), 4 x 8-bit onesweep passes with an "
                  f"atomic look-back across {threads} threads; median of 3 after 1 warm-up; host CPU: {model}",
    }


if __name__ == "__main__":
    main()
