"""Generates the golden fixtures in tests/golden/ from the CPU oracle.

The reference ships no fixtures for this path, so these are produced by the
oracle (oracle/tmac_oracle.c), whose RNG and arithmetic are pinned by
tests/test_oracle.py.  Inputs are regenerated from seeds (the RNG stream is
pinned by known-answer vectors) and a SHA-256 of the input bytes is stored
next to the expected outputs, so a fixture detects both an input drift and an
output drift.  Run:  python tests/golden/gen_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

import oracle  # noqa: E402

NH, NKV, HD = 14, 2, 64
KVD = NKV * HD


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def c1_inputs():
    """Config 1: q [14x64], 256 filled cache rows, query at position 255."""
    q = oracle.normal(10, NH * HD)
    k = oracle.normal(11, (256, KVD))
    v = oracle.normal(12, (256, KVD))
    return q, k, v


def c2_inputs(layers=2, steps=4):
    """Config 2 slice: per (step, layer) pre-RoPE q/k/v, stream 2*1000 + layer."""
    q = np.empty((steps, layers, NH * HD), np.float32)
    kn = np.empty((steps, layers, KVD), np.float32)
    vn = np.empty((steps, layers, KVD), np.float32)
    for layer in range(layers):
        x = oracle.normal(2 * 1000 + layer, steps * (NH * HD + 2 * KVD)).reshape(steps, -1)
        q[:, layer] = x[:, :NH * HD]
        kn[:, layer] = x[:, NH * HD:NH * HD + KVD]
        vn[:, layer] = x[:, NH * HD + KVD:]
    return q, kn, vn


def c2_reference(q, kn, vn, cap=256):
    steps, layers = q.shape[:2]
    kc = np.zeros((layers, cap, KVD), np.float32)
    vc = np.zeros((layers, cap, KVD), np.float32)
    out = np.empty((steps, layers, NH * HD), np.float32)
    for s in range(steps):
        for layer in range(layers):
            out[s, layer], _, _ = oracle.layer_step(q[s, layer], kn[s, layer], vn[s, layer], kc[layer], vc[layer],
                                                    NH, NKV, HD, s, 1e6)
    return out, kc[:, :steps], vc[:, :steps]


def ragged_inputs():
    lens = np.array([1, 3, 16, 17, 100, 513], np.int32)
    offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
    total = int(lens.sum())
    q = oracle.normal(40, (lens.size, NH * HD))
    k = oracle.normal(41, (total, KVD))
    v = oracle.normal(42, (total, KVD))
    return q, k, v, offs, lens


def build() -> dict[str, dict[str, np.ndarray]]:
    fx = {}
    q, k, v = c1_inputs()
    fx["config1"] = {"out": oracle.attention(q, k, v, NH, NKV, HD, 255), "input_sha256": np.array(sha(q, k, v))}
    q, kn, vn = c2_inputs()
    out, kc, vc = c2_reference(q, kn, vn)
    fx["config2_slice"] = {"out": out, "k_rows": kc, "v_rows": vc, "input_sha256": np.array(sha(q, kn, vn))}
    q, k, v, offs, lens = ragged_inputs()
    fx["ragged"] = {"out": oracle.attention_ragged(q, k, v, offs, lens, NH, NKV, HD),
                    "input_sha256": np.array(sha(q, k, v, offs, lens))}
    return fx


def main():
    for name, arrays in build().items():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrays)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
