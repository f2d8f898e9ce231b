"""GPU parity for shapes with no compiled kernel: any GQA group and any even head_dim up to
256 on the reference's dispatch surface (attention_op, rope_op, the fused layer step) and
the fp32 batched / ragged decode.  The reference's attention_op sends head_dim != 64 to
kernel_attn, which takes any group and head_dim (metal_backend.hpp:416-452,
kernel_attn.metal:7-60), and kernel_rope takes any head_dim (kernel_rope.metal:5-22).

Oracle: oracle/tmac_oracle.c (tmac_gguf.cpp:990-1016 RoPE, 1093-1128 attention with the
scale 1/sqrt(head_dim)).  Attention within 2e-5 + 1e-4 |ref|; RoPE and cache rows
bit-exact.  Entry points and cache types that keep head_dim 64 and the compiled groups
must refuse other shapes with TMAC_ERR_UNSUPPORTED."""
import numpy as np
import pytest

import oracle
import tmac_attn
from conftest import assert_close

pytestmark = pytest.mark.gpu

SHAPES = [(3, 1, 64), (6, 3, 64), (14, 2, 32), (14, 2, 128), (8, 8, 80), (12, 4, 96), (2, 1, 2), (5, 5, 256),
          (16, 2, 128), (9, 3, 66)]


@pytest.mark.parametrize("nh,nkv,hd", SHAPES)
@pytest.mark.parametrize("past_len", [0, 5, 255, 1000])
def test_attention_op_any_shape(ctx, nh, nkv, hd, past_len):
    n = past_len + 1
    k = oracle.normal(7000 + hd + past_len, (n, nkv * hd))
    v = oracle.normal(7001 + hd + past_len, (n, nkv * hd))
    q = oracle.normal(7002 + nh + past_len, nh * hd)
    dq, dk, dv, dout = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.empty(nh * hd)
    ctx.attention_op(dq, dk, dv, dout, nh, nkv, hd, past_len)
    assert_close(dout.numpy(), oracle.attention(q, k, v, nh, nkv, hd, past_len),
                 f"attention_op heads {nh}/{nkv} head_dim {hd} past_len {past_len}")
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("hd", [2, 32, 66, 80, 128, 256])
def test_rope_any_head_dim_bit_exact(ctx, hd):
    for n_heads, pos in ((3, 0), (5, 17), (2, 4095), (7, 300000)):
        x = oracle.normal(7100 + hd + pos, n_heads * hd)
        d = ctx.upload(x)
        ctx.rope_op(d, n_heads, hd, pos, 1e6)
        np.testing.assert_array_equal(d.numpy(), oracle.rope_heads(x, n_heads, hd, pos, 1e6))
    rows, stride, n_heads = 9, 4 * hd + 8, 4
    x = oracle.normal(7150 + hd, (rows, stride))
    d = ctx.upload(x)
    ctx.rope_rows(d, rows, stride, n_heads, hd, 100, 1e4)
    got = d.numpy()
    for r in range(rows):
        np.testing.assert_array_equal(got[r, :n_heads * hd], oracle.rope_heads(x[r, :n_heads * hd], n_heads, hd,
                                                                              100 + r, 1e4))
    np.testing.assert_array_equal(got[:, n_heads * hd:], x[:, n_heads * hd:])
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("nh,nkv,hd", [(3, 1, 64), (14, 2, 128), (12, 4, 96), (9, 3, 66)])
def test_batched_and_ragged_any_shape(ctx, nh, nkv, hd):
    n_seq, n_pos = 5, 300
    k = oracle.normal(7200 + hd, (n_seq * n_pos, nkv * hd))
    v = oracle.normal(7201 + hd, (n_seq * n_pos, nkv * hd))
    q = oracle.normal(7202 + hd, (n_seq, nh * hd))
    offs = np.arange(n_seq, dtype=np.int64) * n_pos
    ref = oracle.attention_ragged(q, k, v, offs, np.full(n_seq, n_pos, np.int32), nh, nkv, hd, n_threads=8)
    dq, dk, dv, dout = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.empty((n_seq, nh * hd))
    ctx.decode_batched(dq, dk, dv, dout, n_seq, nh, nkv, hd, n_pos, n_pos)
    assert_close(dout.numpy(), ref, f"batched {nh}/{nkv}/{hd}")
    lens = np.array([1, 0, 300, 77, 2999], np.int32)
    offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
    kr = oracle.normal(7210 + hd, (int(lens.sum()), nkv * hd))
    vr = oracle.normal(7211 + hd, (int(lens.sum()), nkv * hd))
    nz = lens > 0
    ref = np.zeros((lens.size, nh * hd), np.float32)
    ref[nz] = oracle.attention_ragged(q[nz], kr, vr, offs[nz], lens[nz], nh, nkv, hd, n_threads=8)
    dk, dv, do, dl = ctx.upload(kr), ctx.upload(vr), ctx.upload(offs), ctx.upload(lens)
    ctx.decode_ragged(dq, dk, dv, do, dl, dout, lens.size, nh, nkv, hd, 3000)
    assert_close(dout.numpy(), ref, f"ragged {nh}/{nkv}/{hd}")
    ctx.decode_ragged(dq, dk, dv, do, dl, dout, lens.size, nh, nkv, hd, 1000)  # 2999 > max_len: NaN, bit 1
    assert np.all(np.isnan(dout.numpy()[4]))
    assert ctx.check_device_error() == tmac_attn.TMAC_ERR_DEVICE_FAULT
    assert ctx.query_split(4, 300, nh, nkv) == (300, 0)


@pytest.mark.parametrize("nh,nkv,hd", [(3, 1, 64), (14, 2, 128), (8, 8, 80), (9, 3, 66)])
def test_layer_step_any_shape(ctx, nh, nkv, hd):
    """Fused RoPE + cache write + attention, host and device positions, against the
    reference's sequence (tmac_gguf.cpp:1085-1128); cache rows bit-exact."""
    cap = 64
    kc = np.zeros((cap, nkv * hd), np.float32)
    vc = np.zeros((cap, nkv * hd), np.float32)
    dkc, dvc, dout = ctx.upload(kc), ctx.upload(vc), ctx.empty(nh * hd)
    pos_dev = ctx.upload(np.zeros(1, np.int32))
    ctx.rope_prepare(hd, 1e6, cap)
    for pos in range(40):
        q = oracle.normal(7300 + pos, nh * hd)
        kn = oracle.normal(7400 + pos, nkv * hd)
        vn = oracle.normal(7500 + pos, nkv * hd)
        dq, dkn, dvn = ctx.upload(q), ctx.upload(kn), ctx.upload(vn)
        if pos % 2:
            ctx.layer_attention(dq, dkn, dvn, dkc, dvc, dout, nh, nkv, hd, pos, cap, 1e6)
        else:
            pos_dev.copy_from(np.array([pos], np.int32))
            ctx.layer_attention_devpos(dq, dkn, dvn, dkc, dvc, dout, nh, nkv, hd, pos_dev, cap, 1e6)
        ref, _, _ = oracle.layer_step(q, kn, vn, kc, vc, nh, nkv, hd, pos, 1e6)
        assert_close(dout.numpy(), ref, f"layer {nh}/{nkv}/{hd} pos {pos}")
    np.testing.assert_array_equal(dkc.numpy(), kc)
    np.testing.assert_array_equal(dvc.numpy(), vc)
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("nh,nkv,hd", [(2, 1, 2), (14, 2, 32), (14, 2, 128)])
def test_layer_step_any_shape_counter_far_positions(ctx, nh, nkv, hd):
    """A device-side position counter read by the any-shape layer step and moved by
    tmac_pos_update (set, then advanced by one) to positions far past rows * hd / 64
    of a 4096-row RoPE table (127 for hd 2, 2047 for hd 32), up to the last row.  The
    counter first serves a head_dim-64 layer step (whose kernel keeps the counter's
    cached RoPE row), so the advances also refresh that cache from the head_dim-64
    table.  Both layer steps match the oracle (tmac_gguf.cpp:1085-1128) at every
    position, the cache rows bit-exact, and no device error is raised."""
    cap = 4096
    kc = oracle.normal(7600 + hd, (cap, nkv * hd))
    vc = oracle.normal(7601 + hd, (cap, nkv * hd))
    k64 = oracle.normal(7602, (cap, 128))
    v64 = oracle.normal(7603, (cap, 128))
    dkc, dvc, dout = ctx.upload(kc), ctx.upload(vc), ctx.empty(nh * hd)
    dk64, dv64, dout64 = ctx.upload(k64), ctx.upload(v64), ctx.empty(14 * 64)
    pos_dev = ctx.upload(np.zeros(1, np.int32))
    ctx.rope_prepare(hd, 1e6, cap)
    ctx.rope_prepare(64, 1e6, cap)
    s = ctx.stream()
    try:
        for i, (pos, how) in enumerate([(0, "set"), (126, "set"), (127, "add"), (128, "add"), (2046, "set"),
                                        (2047, "add"), (2048, "add"), (4094, "set"), (4095, "add")]):
            if how == "set":
                ctx.pos_update(pos_dev, pos, stream=s)
            else:
                ctx.pos_update(pos_dev, 1, add=True, stream=s)
            q64 = oracle.normal(7610 + i, 14 * 64)
            kn64, vn64 = oracle.normal(7620 + i, 128), oracle.normal(7630 + i, 128)
            q = oracle.normal(7640 + i, nh * hd)
            kn, vn = oracle.normal(7650 + i, nkv * hd), oracle.normal(7660 + i, nkv * hd)
            dq64, dkn64, dvn64 = ctx.upload(q64), ctx.upload(kn64), ctx.upload(vn64)
            dq, dkn, dvn = ctx.upload(q), ctx.upload(kn), ctx.upload(vn)
            ctx.layer_attention_devpos(dq64, dkn64, dvn64, dk64, dv64, dout64, 14, 2, 64, pos_dev, cap, 1e6,
                                       stream=s)
            ctx.layer_attention_devpos(dq, dkn, dvn, dkc, dvc, dout, nh, nkv, hd, pos_dev, cap, 1e6, stream=s)
            ctx.synchronize(s)
            assert int(pos_dev.numpy()[0]) == pos
            ref64, _, _ = oracle.layer_step(q64, kn64, vn64, k64, v64, 14, 2, 64, pos, 1e6)
            ref, _, _ = oracle.layer_step(q, kn, vn, kc, vc, nh, nkv, hd, pos, 1e6)
            assert_close(dout64.numpy(), ref64, f"head_dim 64 layer step at pos {pos}")
            assert_close(dout.numpy(), ref, f"layer {nh}/{nkv}/{hd} pos {pos} ({how})")
            assert ctx.check_device_error() == 0, f"device error at pos {pos}"
            for d in (dq64, dkn64, dvn64, dq, dkn, dvn):
                d.free()
        np.testing.assert_array_equal(dkc.numpy(), kc)
        np.testing.assert_array_equal(dvc.numpy(), vc)
        np.testing.assert_array_equal(dk64.numpy(), k64)
    finally:
        ctx.destroy_stream(s)
        for d in (dkc, dvc, dout, dk64, dv64, dout64, pos_dev):
            d.free()


def test_other_entry_points_refuse_other_shapes(ctx):
    U = tmac_attn.TMAC_ERR_UNSUPPORTED
    d = ctx.empty(1 << 16)
    p = d.ptr
    lib, h = ctx.lib, ctx.handle
    assert lib.tmac_attention_op(h, None, p, p, p, p, 14, 2, 63, 0) == U          # odd head_dim
    assert lib.tmac_attention_op(h, None, p, p, p, p, 2, 1, 258, 0) == U          # above 256
    assert lib.tmac_rope_op(h, None, p, 2, 63, 0, 1e6) == U
    assert lib.tmac_attention_decode_batched_kv(h, None, tmac_attn.TMAC_KV_BF16, p, p, p, p, 1, 14, 2, 128, 8,
                                                8) == U                            # narrow cache: head_dim 64 only
    assert lib.tmac_attention_decode_batched_kv(h, None, tmac_attn.TMAC_KV_Q8_0, p, p, p, p, 1, 3, 1, 64, 8,
                                                8) == U                            # narrow cache: compiled groups only
    assert lib.tmac_attention_prefill(h, None, p, p, p, p, 1, 4, 0, 4, 14, 2, 128) == U
    assert lib.tmac_attention_prefill(h, None, p, p, p, p, 1, 4, 0, 4, 3, 1, 64) == U
    assert lib.tmac_attention_decode_paged(h, None, tmac_attn.TMAC_KV_F32, p, p, p, 1, p, 1, p, p, 1, 3, 1, 64, 16,
                                           0) == U
    d.free()
