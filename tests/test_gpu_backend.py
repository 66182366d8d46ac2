"""The HIP ComputeBackend (oil/backend.h, libmythos_host.so) on the GPU:
tests/backend_test.cpp creates it through ComputeBackend::create as the
reference's tests do (tests/test_all.cpp:244-336), repeats their checks and
holds every vtable operator to closed forms or float64 references; this test
runs it and reports each check."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "bin", "backend_test")


@pytest.mark.gpu
def test_backend_cpp():
    assert os.path.exists(BIN), "tests/bin/backend_test not built (run __graft_entry__.build())"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    fails = [ln for ln in r.stdout.splitlines() if ln.startswith("FAIL")]
    assert r.returncode == 0 and not fails, r.stdout + r.stderr
    assert r.stdout.count("PASS") >= 25
