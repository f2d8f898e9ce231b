"""GPU parity: libtmac_attn.so (through its C ABI) against the CPU oracle.

Oracle = oracle/tmac_oracle.c, the restatement of tmac_gguf.cpp:990-1016 (RoPE),
1090-1091 (cache write) and 1093-1128 (attention).  Tolerance for attention
outputs: |gpu - ref| <= 2e-5 + 1e-4 |ref| elementwise.  RoPE and the cache
write are compared bit for bit.
"""
import ctypes

import numpy as np
import pytest

import oracle
import tmac_attn
from conftest import assert_close

pytestmark = pytest.mark.gpu

KERNELS = {"auto": tmac_attn.TMAC_KERNEL_AUTO, "group": tmac_attn.TMAC_KERNEL_GROUP,
           "head": tmac_attn.TMAC_KERNEL_HEAD, "headv": tmac_attn.TMAC_KERNEL_HEADV}


@pytest.fixture(params=list(KERNELS))
def kernel(request, ctx):
    """Runs the test with the automatic choice and with each decode kernel forced."""
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, KERNELS[request.param])
    yield request.param
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, tmac_attn.TMAC_KERNEL_AUTO)

NH, NKV, HD = 14, 2, 64
KVD = NKV * HD


def rand_cache(seed, n_rows, kvd=KVD):
    return oracle.normal(seed, (n_rows, kvd)), oracle.normal(seed + 1, (n_rows, kvd))


@pytest.mark.parametrize("past_len", [0, 1, 7, 8, 15, 16, 31, 32, 33, 63, 100, 255, 256, 1000, 4095])
def test_attention_op_matches_oracle(ctx, kernel, past_len):
    n_rows = past_len + 1
    k, v = rand_cache(1000 + past_len, n_rows)
    q = oracle.normal(7 + past_len, NH * HD)
    ref = oracle.attention(q, k, v, NH, NKV, HD, past_len)
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    dout = ctx.empty(NH * HD)
    ctx.attention_op(dq, dk, dv, dout, NH, NKV, HD, past_len)
    assert_close(dout.numpy(), ref, f"attention_op past_len={past_len} kernel={kernel}")
    for d in (dq, dk, dv, dout):
        d.free()


def test_attention_op_config1(ctx):
    """Config 1: 14 q heads x 64, 256 filled rows, query at pos 255, seeded N(0,1)."""
    k, v = rand_cache(11, 256)
    q = oracle.normal(10, NH * HD)
    ref = oracle.attention(q, k, v, NH, NKV, HD, 255)
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    dout = ctx.empty(NH * HD)
    ctx.attention_op(dq, dk, dv, dout, NH, NKV, HD, 255)
    assert_close(dout.numpy(), ref, "config1")


@pytest.mark.parametrize("pos", [0, 1, 37, 255, 4095, 32767])
def test_rope_op_bit_exact(ctx, pos):
    q = oracle.normal(20 + pos, NH * HD)
    k = oracle.normal(21 + pos, KVD)
    rq, rk = oracle.rope(q, k, NH, NKV, HD, pos, 1e6)
    dq, dk = ctx.upload(q), ctx.upload(k)
    ctx.rope_op(dq, NH, HD, pos, 1e6)
    ctx.rope_op(dk, NKV, HD, pos, 1e6)
    np.testing.assert_array_equal(dq.numpy(), rq)
    np.testing.assert_array_equal(dk.numpy(), rk)


@pytest.mark.parametrize("n_heads", [NH, NKV])
def test_rope_rows_bit_exact(ctx, n_heads):
    """tmac_rope_rows: 37 rows (padded stride) at positions 1000.. equal
    rope_op / the oracle row by row, bit for bit; the padding is untouched."""
    n_rows, first, stride = 37, 1000, n_heads * HD + 32
    x = oracle.normal(25 + n_heads, (n_rows, stride))
    d = ctx.upload(x)
    ctx.rope_rows(d, n_rows, stride, n_heads, HD, first, 1e6)
    got = d.numpy()
    for r in range(n_rows):
        np.testing.assert_array_equal(got[r, :n_heads * HD], oracle.rope_heads(x[r, :n_heads * HD], n_heads, HD,
                                                                               first + r, 1e6))
    np.testing.assert_array_equal(got[:, n_heads * HD:], x[:, n_heads * HD:])
    assert ctx.check_device_error() == 0


def test_elem_op_cache_write_bit_exact(ctx):
    cache = oracle.normal(30, (256, KVD))
    src = oracle.normal(31, KVD)
    ref = cache.copy()
    oracle.cache_write(ref, 77, src)
    dc, ds = ctx.upload(cache), ctx.upload(src)
    ctx.elem_op(2, dc.at(77 * KVD), ds, KVD)
    np.testing.assert_array_equal(dc.numpy(), ref)


@pytest.mark.parametrize("pos", [0, 1, 8, 31, 32, 33, 200, 255])
def test_layer_attention_matches_reference_sequence(ctx, kernel, pos):
    """Fused launch == rope_op x2 + elem_op(2) x2 + attention_op (tmac_gguf.cpp:1562-1568)."""
    cap = 256
    k_cache = np.zeros((cap, KVD), np.float32)
    v_cache = np.zeros((cap, KVD), np.float32)
    k_cache[:pos], v_cache[:pos] = rand_cache(40 + pos, pos) if pos else (k_cache[:0], v_cache[:0])
    q = oracle.normal(50 + pos, NH * HD)
    kn = oracle.normal(51 + pos, KVD)
    vn = oracle.normal(52 + pos, KVD)
    rk, rv = k_cache.copy(), v_cache.copy()
    ref, _, _ = oracle.layer_step(q, kn, vn, rk, rv, NH, NKV, HD, pos, 1e6)
    dq, dkn, dvn = ctx.upload(q), ctx.upload(kn), ctx.upload(vn)
    dkc, dvc = ctx.upload(k_cache), ctx.upload(v_cache)
    dout = ctx.empty(NH * HD)
    ctx.layer_attention(dq, dkn, dvn, dkc, dvc, dout, NH, NKV, HD, pos, cap, 1e6)
    assert_close(dout.numpy(), ref, f"layer pos={pos} kernel={kernel}")
    np.testing.assert_array_equal(dkc.numpy(), rk)
    np.testing.assert_array_equal(dvc.numpy(), rv)
    np.testing.assert_array_equal(dq.numpy(), q)  # inputs are read only


@pytest.mark.parametrize("n_seq,n_pos", [(1, 1), (3, 17), (8, 513), (32, 4096)])
def test_decode_batched(ctx, kernel, n_seq, n_pos):
    stride = n_pos + 3
    k = oracle.normal(60 + n_pos, (n_seq * stride, KVD))
    v = oracle.normal(61 + n_pos, (n_seq * stride, KVD))
    q = oracle.normal(62 + n_pos, (n_seq, NH * HD))
    offs = np.arange(n_seq, dtype=np.int64) * stride
    lens = np.full(n_seq, n_pos, np.int32)
    ref = oracle.attention_ragged(q, k, v, offs, lens, NH, NKV, HD, n_threads=8)
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    dout = ctx.empty((n_seq, NH * HD))
    ctx.decode_batched(dq, dk, dv, dout, n_seq, NH, NKV, HD, n_pos, stride)
    assert_close(dout.numpy(), ref, f"batched {n_seq}x{n_pos} kernel={kernel}")


def test_decode_ragged(ctx, kernel):
    lens = np.array([1, 2, 9, 16, 17, 300, 2048, 5000, 0, 33], np.int32)
    offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
    total = int(lens.sum())
    k = oracle.normal(70, (total, KVD))
    v = oracle.normal(71, (total, KVD))
    q = oracle.normal(72, (lens.size, NH * HD))
    nz = lens > 0
    ref = np.zeros((lens.size, NH * HD), np.float32)
    ref[nz] = oracle.attention_ragged(q[nz], k, v, offs[nz], lens[nz], NH, NKV, HD, n_threads=8)
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    doff, dlen = ctx.upload(offs), ctx.upload(lens)
    dout = ctx.empty((lens.size, NH * HD))
    for hint in (0, total):  # the split hint changes the schedule, never the result
        dout.fill_bytes(0xFF)
        ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, lens.size, NH, NKV, HD, int(lens.max()), total_rows=hint)
        assert_close(dout.numpy(), ref, f"ragged kernel={kernel} total_rows hint={hint}")
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("waves", [0, 4, 8])
def test_group_kernel_sizes(ctx, waves):
    """The fp32 group kernel with 4- and 8-wave workgroups and the automatic
    choice (4 unless splits would hold under 64 rows): batched shapes on both
    sides of that line, a ragged batch, and the layer step at long context."""
    ctx.set_option(tmac_attn.TMAC_OPT_GROUP_WAVES, waves)
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, tmac_attn.TMAC_KERNEL_GROUP)
    try:
        for n_seq, n_pos in ((1, 4096), (4, 4096), (40, 777)):
            k, v = rand_cache(80 + n_seq, n_seq * n_pos)
            q = oracle.normal(82 + n_seq, (n_seq, NH * HD))
            offs = np.arange(n_seq, dtype=np.int64) * n_pos
            ref = oracle.attention_ragged(q, k, v, offs, np.full(n_seq, n_pos, np.int32), NH, NKV, HD,
                                          n_threads=8)
            dq, dk, dv, dout = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.empty((n_seq, NH * HD))
            ctx.decode_batched(dq, dk, dv, dout, n_seq, NH, NKV, HD, n_pos, n_pos)
            assert_close(dout.numpy(), ref, f"batched {n_seq}x{n_pos} waves={waves}")
            if n_seq == 4:  # the same rows as a ragged batch of unequal lengths
                lens = np.array([4096, 3000, 1, 2500], np.int32)
                dl, do = ctx.upload(lens), ctx.upload(offs)
                ref_r = oracle.attention_ragged(q, k, v, offs, lens, NH, NKV, HD, n_threads=8)
                ctx.decode_ragged(dq, dk, dv, do, dl, dout, n_seq, NH, NKV, HD, 4096, total_rows=int(lens.sum()))
                assert_close(dout.numpy(), ref_r, f"ragged waves={waves}")
        pos, cap = 3000, 3010
        kc, vc = rand_cache(90, cap)
        q, kn, vn = oracle.normal(92, NH * HD), oracle.normal(93, KVD), oracle.normal(94, KVD)
        dq, dkn, dvn = ctx.upload(q), ctx.upload(kn), ctx.upload(vn)
        dkc, dvc, dout = ctx.upload(kc), ctx.upload(vc), ctx.empty(NH * HD)
        ctx.layer_attention(dq, dkn, dvn, dkc, dvc, dout, NH, NKV, HD, pos, cap, 1e6)
        ref, _, _ = oracle.layer_step(q, kn, vn, kc, vc, NH, NKV, HD, pos, 1e6)  # writes row pos of kc, vc
        assert_close(dout.numpy(), ref, f"layer waves={waves}")
        np.testing.assert_array_equal(dkc.numpy(), kc)
        np.testing.assert_array_equal(dvc.numpy(), vc)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_GROUP_WAVES, 0)
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, tmac_attn.TMAC_KERNEL_AUTO)
    assert ctx.check_device_error() == 0


def test_memset_refused_while_capturing(ctx):
    """tmac_memset on a capturing stream returns TMAC_ERR_CAPTURE and records
    nothing; the capture stays usable and the captured RoPE replays exactly."""
    x = oracle.normal(77, 2 * HD)
    d = ctx.upload(x)
    s = ctx.stream()
    ctx.rope_prepare(HD, 1e6, 16)
    ctx.step_begin(s)
    try:
        rc = ctx.lib.tmac_memset(ctx.handle, s, ctypes.c_void_p(d.ptr), 0, d.nbytes)
        assert rc == tmac_attn.TMAC_ERR_CAPTURE
        ctx.rope_op(d, 2, HD, 5, 1e6, stream=s)
    finally:
        g = ctx.step_end(s)
    try:
        ctx.graph_launch(g, s)
        ctx.synchronize(s)
        np.testing.assert_array_equal(d.numpy(), oracle.rope_heads(x, 2, HD, 5, 1e6))
    finally:
        ctx.graph_destroy(g)
        ctx.destroy_stream(s)


def test_graph_24_layer_step_replay(ctx):
    """Config 2 slice: a captured 24-layer step replayed for positions 0..S-1
    with the position read on the device, checked against the oracle per step."""
    L, cap, S = 24, 256, 12
    kc = ctx.upload(np.zeros((L, cap, KVD), np.float32))
    vc = ctx.upload(np.zeros((L, cap, KVD), np.float32))
    ref_k = np.zeros((L, cap, KVD), np.float32)
    ref_v = np.zeros((L, cap, KVD), np.float32)
    dq = ctx.empty((L, NH * HD))
    dkn = ctx.empty((L, KVD))
    dvn = ctx.empty((L, KVD))
    dout = ctx.empty((L, NH * HD))
    pos = ctx.upload(np.zeros(1, np.int32))
    ctx.rope_prepare(HD, 1e6, cap)
    s = ctx.stream()
    # warm the workspace for this shape outside capture
    ctx.layer_attention_devpos(dq.at(0), dkn.at(0), dvn.at(0), kc.at(0), vc.at(0), dout.at(0), NH, NKV,
                               HD, pos, cap, 1e6, stream=s)
    ctx.synchronize(s)
    kc.copy_from(np.zeros((L, cap, KVD), np.float32))
    vc.copy_from(np.zeros((L, cap, KVD), np.float32))
    ctx.step_begin(s)
    for layer in range(L):
        ctx.layer_attention_devpos(dq.at(layer * NH * HD), dkn.at(layer * KVD), dvn.at(layer * KVD),
                                   kc.at(layer * cap * KVD), vc.at(layer * cap * KVD),
                                   dout.at(layer * NH * HD), NH, NKV, HD, pos, cap, 1e6, stream=s)
    ctx.pos_update(pos, 1, add=True, stream=s)
    g = ctx.step_end(s)
    try:
        for step in range(S):
            q = oracle.normal(2000 + step, (L, NH * HD))
            kn = oracle.normal(3000 + step, (L, KVD))
            vn = oracle.normal(4000 + step, (L, KVD))
            dq.copy_from(q)
            dkn.copy_from(kn)
            dvn.copy_from(vn)
            ctx.graph_launch(g, s)
            ctx.synchronize(s)
            got = dout.numpy()
            for layer in range(L):
                ref, _, _ = oracle.layer_step(q[layer], kn[layer], vn[layer], ref_k[layer], ref_v[layer],
                                              NH, NKV, HD, step, 1e6)
                assert_close(got[layer], ref, f"step {step} layer {layer}")
        np.testing.assert_array_equal(kc.numpy(), ref_k)
        np.testing.assert_array_equal(vc.numpy(), ref_v)
        assert int(pos.numpy()[0]) == S
    finally:
        ctx.graph_destroy(g)
        ctx.destroy_stream(s)
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("split", [1, 2, 4, 8])
def test_split_v_head_kernel(ctx, split):
    """The split-V head kernel with each V split: attention_op, a short ragged batch with an
    empty and an over-long sequence, and the layer step at several positions (cache rows
    bit-exact)."""
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, tmac_attn.TMAC_KERNEL_HEADV)
    ctx.set_option(tmac_attn.TMAC_OPT_HV_SPLIT, split)
    try:
        for past_len in (0, 9, 255, 700):
            k, v = rand_cache(1300 + past_len, past_len + 1)
            q = oracle.normal(1301 + past_len, NH * HD)
            dq, dk, dv, dout = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.empty(NH * HD)
            ctx.attention_op(dq, dk, dv, dout, NH, NKV, HD, past_len)
            assert_close(dout.numpy(), oracle.attention(q, k, v, NH, NKV, HD, past_len),
                         f"attention_op split {split} past_len {past_len}")
        lens = np.array([3, 0, 64, 129, 500], np.int32)
        offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
        k, v = rand_cache(1310, int(lens.sum()))
        q = oracle.normal(1311, (lens.size, NH * HD))
        nz = lens > 0
        ref = np.zeros((lens.size, NH * HD), np.float32)
        ref[nz] = oracle.attention_ragged(q[nz], k, v, offs[nz], lens[nz], NH, NKV, HD, n_threads=8)
        dq, dk, dv, do, dl = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.upload(offs), ctx.upload(lens)
        dout = ctx.empty((lens.size, NH * HD))
        ctx.decode_ragged(dq, dk, dv, do, dl, dout, lens.size, NH, NKV, HD, 500)
        assert_close(dout.numpy(), ref, f"ragged split {split}")
        ctx.decode_ragged(dq, dk, dv, do, dl, dout, lens.size, NH, NKV, HD, 200)  # 500 > max_len: NaN, bit 1
        got = dout.numpy()
        assert np.all(np.isnan(got[4])) and np.all(got[1] == 0)
        assert ctx.check_device_error() == tmac_attn.TMAC_ERR_DEVICE_FAULT
        for pos in (0, 1, 100, 255):
            cap = 256
            kc, vc = np.zeros((cap, KVD), np.float32), np.zeros((cap, KVD), np.float32)
            if pos:
                kc[:pos], vc[:pos] = rand_cache(1320 + pos, pos)
            q, kn, vn = oracle.normal(1330 + pos, NH * HD), oracle.normal(1331 + pos, KVD), oracle.normal(1332 + pos, KVD)
            dq, dkn, dvn, dkc, dvc = ctx.upload(q), ctx.upload(kn), ctx.upload(vn), ctx.upload(kc), ctx.upload(vc)
            dout = ctx.empty(NH * HD)
            ctx.layer_attention(dq, dkn, dvn, dkc, dvc, dout, NH, NKV, HD, pos, cap, 1e6)
            ref, _, _ = oracle.layer_step(q, kn, vn, kc, vc, NH, NKV, HD, pos, 1e6)
            assert_close(dout.numpy(), ref, f"layer split {split} pos {pos}")
            np.testing.assert_array_equal(dkc.numpy(), kc)
            np.testing.assert_array_equal(dvc.numpy(), vc)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, tmac_attn.TMAC_KERNEL_AUTO)
        ctx.set_option(tmac_attn.TMAC_OPT_HV_SPLIT, 8)
    assert ctx.check_device_error() == 0
