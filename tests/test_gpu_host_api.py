"""Runs the C++ host-layer test driver (tests/cpp/test_host_api.cpp) on the GPU:
the ops.rs-style C++ wrappers and MoELayer::forward_moe_layer against the oracle."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "test_host_api")


def test_cpp_host_layer():
    assert os.path.exists(BIN), "tests/cpp/test_host_api not built (run __graft_entry__.build())"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "OK: 0 failure(s)" in r.stdout
