"""Runs tests/cpp/test_layer_loop (built by __graft_entry__.build()): the
reference's per-layer attention sequence driven through the hip_backend C++
mirror, checked against the oracle for every layer of every step."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "build", "test_layer_loop")


@pytest.mark.gpu
def test_cpp_layer_loop_driver():
    assert os.path.exists(BIN), "build it with __graft_entry__.build()"
    r = subprocess.run([BIN, "6"], capture_output=True, text=True, timeout=100)
    print(r.stdout[-3000:])
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]
    assert "ALL PASS" in r.stdout
