"""Run-to-run determinism: every entry point, called twice on the same inputs
(and the same options), returns the same bits.

The kernels fix every reduction order: within a wave (DPP and lane-swap trees
of a fixed shape), across the waves of a workgroup (LDS merges in wave order),
and across workgroups (split partials written to fixed workspace slots and
merged by the combine launch in split order; the stream-K schedule cuts the
same ranges for the same lengths).  No floating-point atomic is used, so the
output of a call depends only on its inputs, its shape and the options, not
on which workgroup finished first.  Each case runs the call twice, with other
launches in between so that different workgroups land on different CUs,
and compares the outputs bit for bit (as uint32, so NaN patterns and signed
zeros count too).  Shapes: the BASELINE configs 3, 4 and 5 and the C2 layer
step, plus the paged and narrow-cache variants.
"""
import numpy as np
import pytest

import oracle
import tmac_attn
import workloads
from test_gpu_kv_q8_paged import PR, build_pool, store

pytestmark = pytest.mark.gpu
NH, NKV, HD = 14, 2, 64
QD, KVD = NH * HD, NKV * HD


def bits(dev):
    return dev.numpy().view(np.uint32).copy()


def twice(ctx, call, out, between=None):
    """Runs call(), keeps out's bits, runs `between` (other work), then call()
    again over an output poisoned with 0xFF bytes, and returns both copies."""
    call()
    first = bits(out)
    if between is not None:
        between()
    out.fill_bytes(0xFF)
    call()
    second = bits(out)
    assert ctx.check_device_error() == 0
    return first, second


@pytest.fixture(scope="module")
def c3_dev(ctx):
    q, k, v = workloads.c3(256, 4096)
    d = [ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.empty((256, QD))]
    yield d
    for x in d:
        x.free()


def test_config3_headline_twice(ctx, c3_dev):
    dq, dk, dv, dout = c3_dev
    noise = ctx.empty((64, QD))

    def other():  # a different launch shape in between
        ctx.decode_batched(dq, dk, dv, noise, 64, NH, NKV, HD, 1000, 4096)

    a, b = twice(ctx, lambda: ctx.decode_batched(dq, dk, dv, dout, 256, NH, NKV, HD, 4096, 4096), dout, other)
    np.testing.assert_array_equal(a, b)
    noise.free()


@pytest.mark.parametrize("dt", ["bf16", "q8"])
def test_config3_narrow_caches_twice(ctx, dt):
    q, k, v = workloads.c3(64, 4096)
    if dt == "q8":
        code = tmac_attn.TMAC_KV_Q8_0
        kb = oracle.q8_kv_rows(k.reshape(-1, HD)).reshape(-1, NKV * oracle.Q8_HEAD_BYTES)
        vb = oracle.q8_kv_rows(v.reshape(-1, HD)).reshape(-1, NKV * oracle.Q8_HEAD_BYTES)
    else:
        code = tmac_attn.TMAC_KV_BF16
        kb, vb = store(k, code), store(v, code)
    dq, dk, dv, dout = ctx.upload(q), ctx.upload(kb), ctx.upload(vb), ctx.empty((64, QD))
    a, b = twice(ctx, lambda: ctx.decode_batched(dq, dk, dv, dout, 64, NH, NKV, HD, 4096, 4096, kv_dtype=code),
                 dout, lambda: ctx.decode_batched(dq, dk, dv, dout, 17, NH, NKV, HD, 333, 4096, kv_dtype=code))
    np.testing.assert_array_equal(a, b)
    for x in (dq, dk, dv, dout):
        x.free()


@pytest.mark.parametrize("schedule", ["unit grid, hint", "unit grid", "stream-K"])
def test_config4_twice(ctx, schedule):
    q, k, v, offs, lens = workloads.c4()
    n_seq = lens.size
    dq, dk, dv, doff, dlen = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.upload(offs), ctx.upload(lens)
    dout = ctx.empty((n_seq, QD))
    hint = int(lens.sum()) if schedule == "unit grid, hint" else 0
    ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 2 if schedule == "stream-K" else 0)
    try:
        call = lambda: ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, n_seq, NH, NKV, HD, 32768,  # noqa: E731
                                         total_rows=hint)
        a, b = twice(ctx, call, dout, lambda: ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, 5, NH, NKV, HD,
                                                                32768))
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 1)
    np.testing.assert_array_equal(a, b)
    for x in (dq, dk, dv, doff, dlen, dout):
        x.free()


@pytest.mark.parametrize("dt", [tmac_attn.TMAC_KV_F32, tmac_attn.TMAC_KV_Q8_0])
def test_paged_decode_and_layer_step_twice(ctx, dt):
    lens = np.array([4096, 3000, 1537, 700, 64, 17, 1], np.int32)
    n_seq = lens.size
    rows = [store(oracle.normal(9000 + s, (int(lens[s]), KVD)), dt) for s in range(n_seq)]
    vrows = [store(oracle.normal(9020 + s, (int(lens[s]), KVD)), dt) for s in range(n_seq)]
    n_pages = int(sum((l + PR) // PR for l in lens)) + 3
    kp, table = build_pool(rows, dt, n_pages, np.random.default_rng(90))
    vp, _ = build_pool(vrows, dt, n_pages, np.random.default_rng(90))
    q = oracle.normal(9040, (n_seq, QD))
    dq, dk, dv, dtab, dl = ctx.upload(q), ctx.upload(kp), ctx.upload(vp), ctx.upload(table), ctx.upload(lens)
    dout = ctx.empty((n_seq, QD))
    a, b = twice(ctx, lambda: ctx.decode_paged(dq, dk, dv, n_pages, dtab, table.shape[1], dl, dout, n_seq, NH, NKV,
                                               HD, int(lens.max()), kv_dtype=dt), dout)
    np.testing.assert_array_equal(a, b)
    # the batched paged layer step at the last row of each sequence: it rewrites that row with the same bytes
    positions = (lens - 1).astype(np.int32)
    kn, vn = oracle.normal(9041, (n_seq, KVD)), oracle.normal(9042, (n_seq, KVD))
    dkn, dvn, dpos = ctx.upload(kn), ctx.upload(vn), ctx.upload(positions)
    a, b = twice(ctx, lambda: ctx.layer_attention_paged(dq, dkn, dvn, dk, dv, n_pages, dtab, table.shape[1], dpos,
                                                        dout, n_seq, NH, NKV, HD, int(lens.max()), 1e6,
                                                        kv_dtype=dt), dout)
    np.testing.assert_array_equal(a, b)
    for x in (dq, dk, dv, dtab, dl, dout, dkn, dvn, dpos):
        x.free()


def test_config5_prefill_twice(ctx):
    n_seq, n_q, prefix = 4, 512, 1536
    cap = prefix + n_q
    q, k, v = workloads.c5(n_seq, n_q, prefix)
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    dout = ctx.empty((n_seq, n_q, QD))
    a, b = twice(ctx, lambda: ctx.prefill(dq, dk, dv, dout, n_seq, n_q, prefix, cap, NH, NKV, HD), dout,
                 lambda: ctx.prefill(dq, dk, dv, dout, 1, 77, 100, cap, NH, NKV, HD))
    np.testing.assert_array_equal(a, b)
    tiles = ctx.empty(ctx.prefill_tiles_bytes(n_seq, NKV, cap), np.uint8)
    ctx.prefill_pack_rows(dk, dv, cap, tiles, cap, n_seq, NKV, HD, 0, cap)
    c, d = twice(ctx, lambda: ctx.prefill_tiles(dq, tiles, cap, dout, n_seq, n_q, prefix, NH, NKV, HD), dout)
    np.testing.assert_array_equal(c, d)
    np.testing.assert_array_equal(a, c)  # the tile-copy flow gives the repack-all call's bits
    for x in (dq, dk, dv, dout, tiles):
        x.free()


@pytest.mark.parametrize("pos", [0, 255])
def test_config2_layer_step_twice(ctx, pos):
    """The fused layer step at a given position: it writes row pos (the same
    bytes both times) and attends rows 0..pos."""
    cap = 256
    kc = oracle.normal(9100, (cap, KVD))
    vc = oracle.normal(9101, (cap, KVD))
    q, kn, vn = oracle.normal(9102, QD), oracle.normal(9103, KVD), oracle.normal(9104, KVD)
    dq, dkn, dvn, dk, dv = ctx.upload(q), ctx.upload(kn), ctx.upload(vn), ctx.upload(kc), ctx.upload(vc)
    dout = ctx.empty(QD)
    dpos = ctx.upload(np.array([pos], np.int32))
    ctx.rope_prepare(HD, 1e6, cap)
    a, b = twice(ctx, lambda: ctx.layer_attention(dq, dkn, dvn, dk, dv, dout, NH, NKV, HD, pos, cap), dout)
    np.testing.assert_array_equal(a, b)
    c, d = twice(ctx, lambda: ctx.layer_attention_devpos(dq, dkn, dvn, dk, dv, dout, NH, NKV, HD, dpos, cap), dout)
    np.testing.assert_array_equal(c, d)
    for x in (dq, dkn, dvn, dk, dv, dout, dpos):
        x.free()
