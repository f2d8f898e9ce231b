"""Golden fixtures (tests/golden/*.npz, written by tests/golden/gen_golden.py).

CPU: the oracle reproduces every fixture bit for bit from its seeds.
GPU: libtmac_attn.so matches the stored outputs within 2e-5 + 1e-4|ref|, and
the cache rows written by the fused layer step match bit for bit.
"""
import os
import sys

import numpy as np
import pytest

from conftest import assert_close

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import gen_golden as gg  # noqa: E402

NH, NKV, HD, KVD = gg.NH, gg.NKV, gg.HD, gg.KVD


def load(name):
    with np.load(os.path.join(HERE, "golden", f"{name}.npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_oracle_reproduces_fixtures():
    built = gg.build()
    for name, arrays in built.items():
        stored = load(name)
        assert sorted(stored) == sorted(arrays), name
        for key, val in arrays.items():
            np.testing.assert_array_equal(stored[key], val, err_msg=f"{name}.{key}")


@pytest.mark.gpu
def test_gpu_config1_fixture(ctx):
    fx = load("config1")
    q, k, v = gg.c1_inputs()
    assert gg.sha(q, k, v) == str(fx["input_sha256"])
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    out = ctx.empty(NH * HD)
    ctx.attention_op(dq, dk, dv, out, NH, NKV, HD, 255)
    assert_close(out.numpy(), fx["out"], "config1 fixture")


@pytest.mark.gpu
def test_gpu_config2_slice_fixture(ctx):
    fx = load("config2_slice")
    q, kn, vn = gg.c2_inputs()
    assert gg.sha(q, kn, vn) == str(fx["input_sha256"])
    steps, layers = q.shape[:2]
    cap = 256
    kc = ctx.upload(np.zeros((layers, cap, KVD), np.float32))
    vc = ctx.upload(np.zeros((layers, cap, KVD), np.float32))
    out = ctx.empty(NH * HD)
    for s in range(steps):
        for layer in range(layers):
            dq, dkn, dvn = ctx.upload(q[s, layer]), ctx.upload(kn[s, layer]), ctx.upload(vn[s, layer])
            ctx.layer_attention(dq, dkn, dvn, kc.at(layer * cap * KVD), vc.at(layer * cap * KVD), out,
                                NH, NKV, HD, s, cap, 1e6)
            assert_close(out.numpy(), fx["out"][s, layer], f"config2 step {s} layer {layer}")
    np.testing.assert_array_equal(kc.numpy()[:, :steps], fx["k_rows"])
    np.testing.assert_array_equal(vc.numpy()[:, :steps], fx["v_rows"])


@pytest.mark.gpu
def test_gpu_ragged_fixture(ctx):
    fx = load("ragged")
    q, k, v, offs, lens = gg.ragged_inputs()
    assert gg.sha(q, k, v, offs, lens) == str(fx["input_sha256"])
    dq, dk, dv, do, dl = (ctx.upload(a) for a in (q, k, v, offs, lens))
    out = ctx.empty((lens.size, NH * HD))
    ctx.decode_ragged(dq, dk, dv, do, dl, out, lens.size, NH, NKV, HD, int(lens.max()))
    assert_close(out.numpy(), fx["out"], "ragged fixture")
