"""Runs the C++ drivers under tests/cpp (built by __graft_entry__.build()): the
reference's per-layer attention block (QKV projection + biases, RoPE, cache
write, attention, output projection + residual) driven through the hip_backend
C++ mirror, per op and fused, and a paged Q8_0 serving loop driven through the C
ABI, each checked against the oracle for every layer of every step."""
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


SERVING = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "build", "test_paged_serving")


@pytest.mark.gpu
def test_cpp_paged_serving_driver():
    """A paged Q8_0 serving loop through the C ABI (4 layers x 6 sequences at
    different positions, one captured graph per step, replayed 5 times),
    checked against the oracle per layer and sequence and, at the end, every
    page-pool byte."""
    assert os.path.exists(SERVING), "build it with __graft_entry__.build()"
    r = subprocess.run([SERVING, "5"], capture_output=True, text=True, timeout=100)
    print(r.stdout[-3000:])
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]
    assert "ALL PASS" in r.stdout
