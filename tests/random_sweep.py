#!/usr/bin/env python3
"""Long-run randomized parity sweep over the cases of test_gpu_random_cases.py
(not collected by pytest; needs a GPU and the built library).

    python tests/random_sweep.py --seconds 300 --seed 7 --log2 14 25

Runs each case function with fresh seeds (and sizes log-uniform in
[2^lo, 2^hi)) until the time is up, round-robin over the groups, and prints
one JSON line: cases run per group and the first failures (group, seed,
message).  Exit status 1 when any case failed."""
import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(HERE))


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--seconds", type=float, default=300)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--log2", type=int, nargs=2, default=(0, 22), metavar=("LO", "HI"))
    args = ap.parse_args()
    import torch

    import test_gpu_random_cases as rc

    torch.cuda.set_device(0)
    import lc_parallel_primitive_amd as lcpp

    lcpp.lib()  # fail loudly if the HIP library is missing
    rc.LOG2_RANGE = tuple(args.log2)
    groups = [rc.test_random_reduce_and_scan, rc.test_random_sorts, rc.test_random_by_key, rc.test_random_segments,
              rc.test_random_misaligned_and_variants, rc.test_random_floats]
    counts = {f.__name__: 0 for f in groups}
    failures = []
    end = time.time() + args.seconds
    k = 0
    while time.time() < end:
        f = groups[k % len(groups)]
        seed = 1_000_000 * args.seed + k
        try:
            f(None, seed)
        except AssertionError as exc:
            failures.append((f.__name__, seed, str(exc)[:200]))
            print(f"FAIL {f.__name__} seed={seed} {str(exc)[:200]}", flush=True)
        counts[f.__name__] += 1
        k += 1
        if k % 50 == 0:
            print(f"[sweep] {k} cases, {len(failures)} failures", flush=True)
    print(json.dumps({"cases": counts, "failures": len(failures), "first": failures[:5],
                      "log2": list(args.log2), "seed": args.seed}), flush=True)
    return 1 if failures else 0


if __name__ == "__main__":
    sys.exit(main())
