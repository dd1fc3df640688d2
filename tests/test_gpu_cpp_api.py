"""The reference's C++ API (include/lcpp/parallel_primitive.h) end to end:
tests/cpp/reference_style_test.cpp drives DeviceReduce / DeviceScan /
DeviceRadixSort / DeviceSegmentReduce the way the reference's own tests do,
on the GPU, through liblcpp_amd.so."""
import os
import subprocess

import pytest

from conftest import ROOT, log

pytestmark = pytest.mark.gpu

BIN = os.path.join(ROOT, "tests", "cpp", "reference_style_test")


def test_cpp_reference_style_program(gpu):
    assert os.path.exists(BIN), f"{BIN} missing: run __graft_entry__.build()"
    log("C++ reference-style program")
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=90)
    print(r.stdout)
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith(("ok ", "FAIL "))]
    assert r.returncode == 0, r.stdout + r.stderr
    assert len(lines) >= 18 and all(ln.startswith("ok ") for ln in lines)
    assert "PASSED: 0 failure(s)" in r.stdout
