"""CPU-tier sanitizer runs (built by oracle/Makefile, outputs in oracle/_san/).

- The CPU oracle under ASan + UBSan, and under TSan: the multithreaded
  look-back restatements (the KAT, the bounded wait with a withheld
  predecessor, the single-pass scan, the onesweep sort passes) and the
  multithreaded reduce / segment reduce, cross-checked against the
  single-threaded functions by oracle/san/oracle_check.c.
- A TSan build with a planted race (a publish without release ordering):
  its run must report the race, so a clean TSan run means something.
- The C ABI's host code, compiled from the library's own sources with the
  sanitizers on the host side only, under ASan + UBSan: every temp-size
  query over all dtypes and sizes up to 2^64-1, and every entry point with
  one invalid argument at a time (oracle/san/capi_args.cpp).  Nothing here
  touches a GPU."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle")
SAN = os.path.join(ORACLE, "_san")


def _make(target, timeout):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    r = subprocess.run(["make", "-s", "-j8", "-C", ORACLE, target], capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, r.stdout + r.stderr


def _run(exe, *args, env=None, timeout=600):
    e = dict(os.environ)
    e.update(env or {})
    return subprocess.run([os.path.join(SAN, exe), *args], capture_output=True, text=True, timeout=timeout, env=e)


def test_oracle_asan_ubsan():
    _make("_san/oracle_asan", 300)
    r = _run("oracle_asan")
    assert r.returncode == 0 and "oracle_check: OK" in r.stdout, r.stdout + r.stderr[-4000:]


def test_oracle_tsan_lookback_restatements():
    _make("_san/oracle_tsan", 300)
    r = _run("oracle_tsan", env={"TSAN_OPTIONS": "halt_on_error=1"})
    assert r.returncode == 0 and "oracle_check: OK" in r.stdout, r.stdout + r.stderr[-4000:]
    assert "ThreadSanitizer" not in r.stderr


def test_tsan_reports_planted_race():
    _make("_san/oracle_tsan_planted", 300)
    r = _run("oracle_tsan_planted", "reduce", env={"TSAN_OPTIONS": "halt_on_error=1"})
    assert r.returncode != 0
    assert "ThreadSanitizer: data race" in r.stderr and "scan_mt_worker" in r.stderr


def test_capi_host_asan_ubsan():
    if not os.path.exists("/opt/rocm/bin/hipcc") and shutil.which("hipcc") is None:
        pytest.skip("hipcc not available")
    _make("_san/capi_asan", 900)
    r = _run("capi_asan", env={"ASAN_OPTIONS": "detect_leaks=0"})
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]
    if "capi_args: OK" not in r.stdout:
        # capi_args sweeps the argument checks only where no GPU is visible
        assert "skipped" in r.stdout, r.stdout
        pytest.skip("capi_args: a GPU is visible, so the argument sweep did not run")
