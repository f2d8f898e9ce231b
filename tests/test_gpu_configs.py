"""GPU parity at the exact benchmark configurations, through the C ABI.

Each test runs the launch the benchmark times, on the inputs the benchmark
draws (tmac_gguf.cpp_amd/workloads.py), and compares every output with the
oracle (oracle/tmac_oracle.c, the restatement of tmac_gguf.cpp:990-1016 RoPE,
1090-1091 cache write and 1093-1128 attention).  Tolerance for attention
outputs: |gpu - ref| <= 2e-5 + 1e-4 |ref| elementwise; cache rows bit-exact.
"""
import numpy as np
import pytest

import oracle
import workloads
from conftest import assert_close

pytestmark = pytest.mark.gpu
NH, NKV, HD = 14, 2, 64
QD, KVD = NH * HD, NKV * HD


def bf16_round(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


def test_config3_headline_launch(ctx):
    """Config 3: 256 sequences x 4096 rows.  On MI355X's 256 CUs the automatic
    schedule is one split per sequence (the 4-wave group kernel writing the
    output directly, no combine); all 256 sequences are checked."""
    n_seq, n_pos = 256, 4096
    info, n_cu = ctx.device_info()
    split = ctx.query_split(n_seq, n_pos, NH, NKV)
    if n_cu == 256:
        assert split == (4096, 1), split
    q, k, v = workloads.c3(n_seq, n_pos)
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    dout = ctx.empty((n_seq, QD))
    dout.fill_bytes(0xFF)
    ctx.decode_batched(dq, dk, dv, dout, n_seq, NH, NKV, HD, n_pos, n_pos)
    got = dout.numpy()
    for d in (dq, dk, dv, dout):
        d.free()
    offs = np.arange(n_seq, dtype=np.int64) * n_pos
    ref = oracle.attention_ragged(q, k, v, offs, np.full(n_seq, n_pos, np.int32), NH, NKV, HD, n_threads=16)
    assert_close(got, ref, f"config 3 {n_seq}x{n_pos} split {split}")
    assert ctx.check_device_error() == 0


def test_config4_ragged(ctx):
    """Config 4: 16 sequences with lengths 1 + floor(u * 32768) from the seeded
    uniform stream, packed pool, default schedule, with and without the
    total_rows hint the benchmark passes; all 16 outputs checked."""
    q, k, v, offs, lens = workloads.c4()
    total = int(lens.sum())
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    doff, dlen = ctx.upload(offs), ctx.upload(lens)
    dout = ctx.empty((lens.size, QD))
    ref = oracle.attention_ragged(q, k, v, offs, lens, NH, NKV, HD, n_threads=16)
    for hint in (total, 0):
        dout.fill_bytes(0xFF)
        ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, lens.size, NH, NKV, HD, 32768, total_rows=hint)
        assert_close(dout.numpy(), ref, f"config 4 total_rows={hint} ({total} rows)")
    for d in (dq, dk, dv, doff, dlen, dout):
        d.free()
    assert ctx.check_device_error() == 0


def test_config2_full_sweep_graph(ctx):
    """Config 2: the captured 24-layer step (one fused layer launch per layer
    plus the position advance) replayed for every position 0..255 of a zeroed
    256-row cache; every layer's output of every step against the oracle, and
    both caches bit-exact at the end."""
    L, cap = 24, 256
    q, kn, vn = workloads.c2(L, cap)
    kc = ctx.upload(np.zeros((L, cap, KVD), np.float32))
    vc = ctx.upload(np.zeros((L, cap, KVD), np.float32))
    ref_k = np.zeros((L, cap, KVD), np.float32)
    ref_v = np.zeros((L, cap, KVD), np.float32)
    dq, dkn, dvn, dout = ctx.empty((L, QD)), ctx.empty((L, KVD)), ctx.empty((L, KVD)), ctx.empty((L, QD))
    pos = ctx.upload(np.zeros(1, np.int32))
    ctx.rope_prepare(HD, 1e6, cap)
    s = ctx.stream()

    def layer(i):
        ctx.layer_attention_devpos(dq.at(i * QD), dkn.at(i * KVD), dvn.at(i * KVD), kc.at(i * cap * KVD),
                                   vc.at(i * cap * KVD), dout.at(i * QD), NH, NKV, HD, pos, cap, 1e6, stream=s)

    ctx.step_begin(s)
    for i in range(L):
        layer(i)
    ctx.pos_update(pos, 1, add=True, stream=s)
    g = ctx.step_end(s)
    worst = 0.0
    try:
        for step in range(cap):
            dq.copy_from(q[step])
            dkn.copy_from(kn[step])
            dvn.copy_from(vn[step])
            ctx.graph_launch(g, s)
            ctx.synchronize(s)
            got = dout.numpy()
            for i in range(L):
                ref, _, _ = oracle.layer_step(q[step, i], kn[step, i], vn[step, i], ref_k[i], ref_v[i],
                                              NH, NKV, HD, step, 1e6)
                worst = max(worst, assert_close(got[i], ref, f"config 2 step {step} (pos {step}) layer {i}"))
        np.testing.assert_array_equal(kc.numpy(), ref_k)
        np.testing.assert_array_equal(vc.numpy(), ref_v)
        assert int(pos.numpy()[0]) == cap
    finally:
        ctx.graph_destroy(g)
        ctx.destroy_stream(s)
        for d in (kc, vc, dq, dkn, dvn, dout, pos):
            d.free()
    print(f"config 2 full sweep: max abs err {worst:.3e}")
    assert ctx.check_device_error() == 0


def test_config5_all_rows(ctx):
    """Config 5: 4 sequences, 512-query chunk after a 1536-row prefix, raw fp32
    inputs (the kernel rounds them to bf16); all 4 x 512 query rows against the
    oracle on the bf16-rounded inputs."""
    n_seq, n_q, prefix = 4, 512, 1536
    cap = prefix + n_q
    q, k, v = workloads.c5(n_seq, n_q, prefix)
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    dout = ctx.empty((n_seq, n_q, QD))
    ctx.prefill(dq, dk, dv, dout, n_seq, n_q, prefix, cap, NH, NKV, HD)
    got = dout.numpy()
    for d in (dq, dk, dv, dout):
        d.free()
    ref = oracle.prefill(bf16_round(q), bf16_round(k), bf16_round(v), n_seq, n_q, prefix, cap, NH, NKV, HD,
                         n_threads=16)
    assert_close(got, ref, "config 5 all rows")


def test_graph_replay_after_workspace_growth():
    """A graph captured with the split-KV workspace at one size keeps replaying
    exactly after an eager call has made the context grow its workspace (the
    old buffer stays allocated while the graph lives).  A fresh context, so the
    workspace starts at its initial size."""
    import tmac_attn
    with tmac_attn.Context(0) as ctx:
        _workspace_growth(ctx)


def _workspace_growth(ctx):
    import tmac_attn
    n_seq, n_pos = 2, 3000
    q, k, v = workloads.c3(n_seq, n_pos)
    dq, dk, dv, dout = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.empty((n_seq, QD))
    offs = np.arange(n_seq, dtype=np.int64) * n_pos
    ref = oracle.attention_ragged(q, k, v, offs, np.full(n_seq, n_pos, np.int32), NH, NKV, HD, n_threads=8)
    s = ctx.stream()
    ctx.decode_batched(dq, dk, dv, dout, n_seq, NH, NKV, HD, n_pos, n_pos, stream=s)  # sizes the workspace
    ctx.synchronize(s)
    ctx.step_begin(s)
    ctx.decode_batched(dq, dk, dv, dout, n_seq, NH, NKV, HD, n_pos, n_pos, stream=s)
    g = ctx.step_end(s)
    try:
        # an eager ragged call whose partials need far more workspace than any call so far
        n_big, rows_big = 4000, 64
        lens = np.full(n_big, rows_big, np.int32)
        kb = oracle.normal(9901, (n_big * rows_big, KVD))
        vb = oracle.normal(9902, (n_big * rows_big, KVD))
        qb = oracle.normal(9903, (n_big, QD))
        ob = np.arange(n_big, dtype=np.int64) * rows_big
        dkb, dvb, dqb, dob, dlb = ctx.upload(kb), ctx.upload(vb), ctx.upload(qb), ctx.upload(ob), ctx.upload(lens)
        doutb = ctx.empty((n_big, QD))
        ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 2)
        try:
            ctx.decode_ragged(dqb, dkb, dvb, dob, dlb, doutb, n_big, NH, NKV, HD, rows_big, stream=s)
        finally:
            ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 1)
        ctx.synchronize(s)
        refb = oracle.attention_ragged(qb, kb, vb, ob, lens, NH, NKV, HD, n_threads=16)
        assert_close(doutb.numpy(), refb, "eager call that grew the workspace")
        for rep in range(3):
            dout.fill_bytes(0xFF, s)
            ctx.graph_launch(g, s)
            ctx.synchronize(s)
            assert_close(dout.numpy(), ref, f"replay {rep} after the workspace grew")
        for d in (dkb, dvb, dqb, dob, dlb, doutb):
            d.free()
    finally:
        ctx.graph_destroy(g)
        ctx.destroy_stream(s)
        for d in (dq, dk, dv, dout):
            d.free()
    assert ctx.check_device_error() == 0


def test_graph_replay_after_rope_table_growth():
    """The same for the RoPE table: a captured rope_op keeps its table after an
    eager call at a far position has replaced it with a larger one."""
    import tmac_attn
    with tmac_attn.Context(0) as ctx:
        x = oracle.normal(9911, QD)
        d = ctx.upload(x)
        ctx.rope_prepare(HD, 1e6, 16)
        s = ctx.stream()
        ctx.step_begin(s)
        ctx.rope_op(d, NH, HD, 5, 1e6, stream=s)
        g = ctx.step_end(s)
        try:
            far = ctx.upload(x)
            ctx.rope_op(far, NH, HD, 300000, 1e6, stream=s)  # the table grows to cover position 300000
            ctx.synchronize(s)
            np.testing.assert_array_equal(far.numpy(), oracle.rope_heads(x, NH, HD, 300000, 1e6))
            for rep in range(3):
                d.copy_from(x)
                ctx.graph_launch(g, s)
                ctx.synchronize(s)
                np.testing.assert_array_equal(d.numpy(), oracle.rope_heads(x, NH, HD, 5, 1e6), f"replay {rep}")
        finally:
            ctx.graph_destroy(g)
            ctx.destroy_stream(s)
        assert ctx.check_device_error() == 0
