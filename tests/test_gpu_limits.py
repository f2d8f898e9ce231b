"""GPU parity at the limits of the decode entry points: the split cap
(kMaxSplits = 256 workgroups per sequence, merged in chunks of 32), thousands
of ragged sequences (the unit scan walks the lengths 64 at a time), row and
page indices whose byte addresses exceed 2^32 (64-bit address arithmetic),
and the sequence-count limit of the launch grid.

Contract as everywhere: |gpu - ref| <= 2e-5 + 1e-4 |ref| against the oracle's
attention (tmac_gguf.cpp:1093-1128) on the same rows.  One exception, the
65,613-row sequence: there the oracle's own fp32 sums (one sequential sum of
65K exponentials, then one of 65K weighted rows, as tmac_gguf.cpp:1116-1126
does them) are up to 1.6e-4 from the exact softmax, outside that bar by
themselves, so the GPU is held to the bar against a float64 evaluation of the
same softmax, and the oracle to its own float64 distance.
"""
import ctypes

import numpy as np
import pytest

import oracle
import tmac_attn
from conftest import assert_close

pytestmark = pytest.mark.gpu
NH, NKV, HD = 14, 2, 64
KVD = NKV * HD
PR = tmac_attn.PAGE_ROWS


def attention_f64(q, k, v, n_head=NH, n_kv_head=NKV):
    """Softmax attention of one query row over all rows, in float64 (the
    closed form the fp32 evaluations approximate)."""
    n = k.shape[0]
    k64 = np.asarray(k, np.float64).reshape(n, n_kv_head, HD)
    v64 = np.asarray(v, np.float64).reshape(n, n_kv_head, HD)
    q64 = np.asarray(q, np.float64).reshape(n_head, HD)
    out = np.empty((n_head, HD))
    g = n_head // n_kv_head
    for h in range(n_head):
        s = k64[:, h // g, :] @ q64[h] / 8.0
        p = np.exp(s - s.max())
        out[h] = (p[:, None] * v64[:, h // g, :]).sum(0) / p.sum()
    return out.reshape(1, n_head * HD)


def put_rows(ctx, dst, row, host):
    """Copies host rows [n, KVD] (fp32) into device array `dst` at row `row`."""
    host = np.ascontiguousarray(host, np.float32)
    rc = ctx.lib.tmac_memcpy_h2d(ctx.handle, None, ctypes.c_void_p(dst.at(row * KVD)),
                                 ctypes.c_void_p(host.ctypes.data), host.nbytes)
    assert rc == 0, tmac_attn.status_string(rc)


@pytest.mark.parametrize("dt", [tmac_attn.TMAC_KV_F32, tmac_attn.TMAC_KV_BF16])
def test_split_cap_single_long_sequence(ctx, dt):
    """One 65,613-row sequence with a requested 16-row split: the split length
    grows until at most 256 splits remain, and the combine merges them in 8
    chunks of 32 with a running max (rows of very different magnitudes move
    the max between chunks)."""
    n_pos = 65536 + 77
    rng = np.random.default_rng(5)
    scale = np.exp2(rng.uniform(-2, 2, (n_pos, 1))).astype(np.float32)
    k = oracle.normal(3100, (n_pos, KVD)) * scale
    v = oracle.normal(3101, (n_pos, KVD))
    q = oracle.normal(3102, (1, NH * HD))
    if dt == tmac_attn.TMAC_KV_BF16:  # the cache holds bf16: compare against the widened rows
        def rnd(x):
            u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
            bits = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)
            return bits, (bits.astype(np.uint32) << 16).view(np.float32)
        kb, k = rnd(k)
        vb, v = rnd(v)
    else:
        kb, vb = k, v
    dq, dk, dv, dout = ctx.upload(q), ctx.upload(kb), ctx.upload(vb), ctx.empty((1, NH * HD))
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, tmac_attn.TMAC_KERNEL_GROUP)
    ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 16)
    try:
        split_len, n_splits = ctx.query_split(1, n_pos, NH, NKV)
        assert n_splits <= 256 and split_len * n_splits >= n_pos, (split_len, n_splits)
        assert n_splits > 200, n_splits
        ctx.decode_batched(dq, dk, dv, dout, 1, NH, NKV, HD, n_pos, n_pos, kv_dtype=dt)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 0)
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, 0)
    got = dout.numpy()
    exact = attention_f64(q, k, v)
    assert_close(got, exact, f"split cap dt={dt} against float64")
    ref = oracle.attention_ragged(q, k, v, np.zeros(1, np.int64), np.array([n_pos], np.int32), NH, NKV, HD)
    oracle_dev = np.abs(ref - exact)
    assert oracle_dev.max() < 5e-4  # the oracle's fp32 sums at 65K rows (1.6e-4 measured)
    assert np.all(np.abs(got - ref) <= oracle_dev + 2e-5 + 1e-4 * np.abs(exact))
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("paged", [False, True])
def test_thousands_of_ragged_sequences(ctx, paged):
    """3,000 sequences of 0..40 rows, ragged and paged: the unit scan over the
    lengths runs 47 chunks of 64, and empty sequences give zero outputs."""
    n_seq = 3000
    rng = np.random.default_rng(6)
    lens = rng.integers(0, 41, n_seq).astype(np.int32)
    lens[:5] = [0, 1, 40, 0, 16]
    offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
    rows = int(lens.sum())
    k, v = oracle.normal(3200, (rows, KVD)), oracle.normal(3201, (rows, KVD))
    q = oracle.normal(3202, (n_seq, NH * HD))
    dq, dl, dout = ctx.upload(q), ctx.upload(lens), ctx.empty((n_seq, NH * HD))
    dout.fill_bytes(0xFF)
    if paged:
        max_pages = (int(lens.max()) + PR - 1) // PR
        n_pages = int(sum((l + PR - 1) // PR for l in lens)) + 7
        perm = rng.permutation(n_pages)
        table = np.zeros((n_seq, max_pages), np.int32)
        kp = np.zeros((n_pages * PR, KVD), np.float32)
        vp = np.zeros((n_pages * PR, KVD), np.float32)
        nxt = 0
        for s in range(n_seq):
            for j in range((lens[s] + PR - 1) // PR):
                pg = perm[nxt]
                nxt += 1
                table[s, j] = pg
                seg = slice(offs[s] + j * PR, offs[s] + min(lens[s], (j + 1) * PR))
                kp[pg * PR:pg * PR + seg.stop - seg.start] = k[seg]
                vp[pg * PR:pg * PR + seg.stop - seg.start] = v[seg]
        dk, dv, dt_ = ctx.upload(kp), ctx.upload(vp), ctx.upload(table)
        ctx.decode_paged(dq, dk, dv, n_pages, dt_, max_pages, dl, dout, n_seq, NH, NKV, HD, int(lens.max()),
                         total_rows=rows)
    else:
        dk, dv, do = ctx.upload(k), ctx.upload(v), ctx.upload(offs)
        ctx.decode_ragged(dq, dk, dv, do, dl, dout, n_seq, NH, NKV, HD, int(lens.max()), total_rows=rows)
    got = dout.numpy()
    nz = lens > 0
    assert np.all(got[~nz] == 0)
    ref = oracle.attention_ragged(q[nz], k, v, offs[nz], lens[nz], NH, NKV, HD, n_threads=8)
    assert_close(got[nz], ref, f"{n_seq} ragged sequences paged={paged}")
    assert ctx.check_device_error() == 0


def test_byte_offsets_above_4gib(ctx):
    """K/V pools of 9,000,000 fp32 rows (4.6 GB each): ragged sequences and a
    batched stride whose rows start past byte 2^32, and pages whose index
    times the page bytes passes 2^32."""
    cap = 9_000_000
    dk, dv = ctx.empty((cap, KVD)), ctx.empty((cap, KVD))
    try:
        # ragged: sequences at rows 8,400,000 / 100 / 8,990,000
        lens = np.array([3000, 500, 5000], np.int32)
        offs = np.array([8_400_000, 100, 8_990_000], np.int64)
        k = oracle.normal(3300, (int(lens.sum()), KVD))
        v = oracle.normal(3301, (int(lens.sum()), KVD))
        host_offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
        for o, ho, n in zip(offs, host_offs, lens):
            put_rows(ctx, dk, int(o), k[ho:ho + n])
            put_rows(ctx, dv, int(o), v[ho:ho + n])
        q = oracle.normal(3302, (3, NH * HD))
        dq, dout = ctx.upload(q), ctx.empty((3, NH * HD))
        ctx.decode_ragged(dq, dk, dv, ctx.upload(offs), ctx.upload(lens), dout, 3, NH, NKV, HD, 5000)
        ref = oracle.attention_ragged(q, k, v, host_offs, lens, NH, NKV, HD, n_threads=8)
        assert_close(dout.numpy(), ref, "ragged rows past 2^32 bytes")
        # batched: stride 4,400,000 rows, so sequence 2 starts at byte 4.5e9 (rows 8,800,000..)
        n_pos, stride = 1200, 4_400_000
        kb, vb = oracle.normal(3303, (3 * n_pos, KVD)), oracle.normal(3304, (3 * n_pos, KVD))
        for s in range(3):
            put_rows(ctx, dk, s * stride, kb[s * n_pos:(s + 1) * n_pos])
            put_rows(ctx, dv, s * stride, vb[s * n_pos:(s + 1) * n_pos])
        ctx.decode_batched(dq, dk, dv, dout, 3, NH, NKV, HD, n_pos, stride)
        ref = oracle.attention_ragged(q, kb, vb, np.arange(3, dtype=np.int64) * n_pos,
                                      np.full(3, n_pos, np.int32), NH, NKV, HD, n_threads=8)
        assert_close(dout.numpy(), ref, "batched stride past 2^32 bytes")
        # paged: pool pages 562,000 + (0..), i.e. rows from 8,992,000 (byte 4.6e9)
        n_pages = cap // PR
        lp = np.array([700, 33], np.int32)
        max_pages = (int(lp.max()) + PR - 1) // PR
        table = np.zeros((2, max_pages), np.int32)
        kq, vq = oracle.normal(3305, (int(lp.sum()), KVD)), oracle.normal(3306, (int(lp.sum()), KVD))
        hoff = np.array([0, 700], np.int64)
        nxt = n_pages - 1
        for s in range(2):
            for j in range((lp[s] + PR - 1) // PR):
                table[s, j] = nxt
                seg = slice(hoff[s] + j * PR, hoff[s] + min(lp[s], (j + 1) * PR))
                put_rows(ctx, dk, nxt * PR, kq[seg])
                put_rows(ctx, dv, nxt * PR, vq[seg])
                nxt -= 1
        dout2 = ctx.empty((2, NH * HD))
        ctx.decode_paged(dq, dk, dv, n_pages, ctx.upload(table), max_pages, ctx.upload(lp), dout2, 2, NH, NKV, HD,
                         int(lp.max()))
        ref = oracle.attention_ragged(q[:2], kq, vq, hoff, lp, NH, NKV, HD, n_threads=8)
        assert_close(dout2.numpy(), ref, "pages past 2^32 bytes")
        assert ctx.check_device_error() == 0
    finally:
        dk.free()
        dv.free()


def test_sequence_count_limit(ctx):
    """The (split, sequence) grid holds at most 65,535 sequences: more is
    rejected before any launch."""
    d = ctx.empty(64)
    rc = ctx.decode_batched(d, d, d, d, 65536, NH, NKV, HD, 16, 16, check=False)
    assert rc == tmac_attn.TMAC_ERR_INVALID_ARG
