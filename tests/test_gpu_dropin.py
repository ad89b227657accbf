"""GPU test of the C++ drop-in boundary: runs tests/cpp/kernel_test_dropin,
the reference kernel test's blocks (src/TwoStage/kernel_test.cpp:210-441)
called through the two_stage_cuda:: / linear_cuda:: wrappers of
include/cxxgpt_dropin.hpp, every comparison asserted against the C oracle."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "kernel_test_dropin")


def test_kernel_test_dropin(dev):
    assert os.path.exists(BIN), "tests/cpp/kernel_test_dropin not built (run __graft_entry__.build())"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASSED" in r.stdout
