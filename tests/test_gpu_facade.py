"""The C++ drop-in (libmythos_host.so) on the GPU: tests/facade_test.cpp calls
oil::kernel::* with host pointers and oil::Tensor exactly as the reference's
callers do and checks exact closed forms; this test runs it and reports each
check."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "bin", "facade_test")


@pytest.mark.gpu
def test_facade_cpp():
    assert os.path.exists(BIN), "tests/bin/facade_test not built (run __graft_entry__.build())"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    fails = [ln for ln in r.stdout.splitlines() if ln.startswith("FAIL")]
    assert r.returncode == 0 and not fails, r.stdout + r.stderr
    assert r.stdout.count("PASS") >= 11
