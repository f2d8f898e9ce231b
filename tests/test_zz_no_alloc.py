"""The ragged decode entry point that allocates nothing
(tmac_attention_decode_ragged_noalloc), through the C ABI.

Its output must equal tmac_attention_decode_ragged's (the same kernels and
schedule, only the split-KV partials in the fixed scratch array) bit for bit,
and the oracle (tmac_gguf.cpp:1093-1128 per sequence) within 2e-5 + 1e-4 |ref|;
on two calls in a row, the second one smaller, under both schedules.  A batch
whose partials exceed the fixed array is refused before any launch.
"""

import numpy as np
import pytest

import oracle
import tmac_attn
import workloads
from conftest import assert_close

pytestmark = pytest.mark.gpu
NH, NKV, HD = 14, 2, 64
QD, KVD = NH * HD, NKV * HD


def ragged(ctx, lens, seed):
    lens = np.asarray(lens, np.int32)
    offs = np.concatenate([[0], np.cumsum(lens[:-1], dtype=np.int64)]).astype(np.int64)
    total = int(lens.sum())
    q = oracle.normal(seed, (lens.size, QD))
    k = oracle.normal(seed + 1, (max(total, 1), KVD))
    v = oracle.normal(seed + 2, (max(total, 1), KVD))
    nz = lens > 0
    ref = np.zeros((lens.size, QD), np.float32)
    ref[nz] = oracle.attention_ragged(q[nz], k, v, offs[nz], lens[nz], NH, NKV, HD, n_threads=16)
    dev = [ctx.upload(a) for a in (q, k, v, offs, lens)] + [ctx.empty((lens.size, QD)), ctx.empty((lens.size, QD))]
    return dev, ref, int(lens.max()), total


def call_noalloc(ctx, dev, n_seq, max_len, total):
    dq, dk, dv, doff, dlen, dout, _ = dev
    return ctx.lib.tmac_attention_decode_ragged_noalloc(ctx.handle, None, dq.ptr, dk.ptr, dv.ptr, doff.ptr, dlen.ptr,
                                                        dout.ptr, n_seq, NH, NKV, HD, max_len, total)


def call_alloc(ctx, dev, n_seq, max_len, total):
    dq, dk, dv, doff, dlen, _, dout = dev
    return ctx.lib.tmac_attention_decode_ragged(ctx.handle, None, dq.ptr, dk.ptr, dv.ptr, doff.ptr, dlen.ptr,
                                                dout.ptr, n_seq, NH, NKV, HD, max_len, total)


@pytest.mark.parametrize("stream_k", [0, 2])
def test_noalloc_matches_allocating_entry_point(ctx, stream_k):
    ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, stream_k)
    try:
        q4, k4, v4, offs4, lens4 = workloads.c4()  # config 4: 16 sequences up to 32,768 rows
        big = [ctx.upload(a) for a in (q4, k4, v4, offs4, lens4)] + [ctx.empty((16, QD)), ctx.empty((16, QD))]
        ref4 = oracle.attention_ragged(q4, k4, v4, offs4, lens4, NH, NKV, HD, n_threads=16)
        small, ref_s, max_s, total_s = ragged(ctx, [5, 0, 1500, 3000, 1], 9300)
        cases = [(big, ref4, 16, 32768, int(lens4.sum())), (small, ref_s, 5, max_s, total_s)]
        for i, (dev, ref, n_seq, max_len, total) in enumerate(cases):  # the second call is the smaller
            dev[5].fill_bytes(0xFF)
            dev[6].fill_bytes(0xFF)
            assert call_noalloc(ctx, dev, n_seq, max_len, total) == tmac_attn.TMAC_OK, ctx.lib.tmac_last_error(ctx.handle).decode()
            assert call_alloc(ctx, dev, n_seq, max_len, total) == tmac_attn.TMAC_OK, ctx.lib.tmac_last_error(ctx.handle).decode()
            got, want = dev[5].numpy(), dev[6].numpy()
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32),
                                          err_msg=f"call {i}: noalloc vs allocating entry point")
            assert_close(got, ref, f"call {i} stream_k={stream_k} vs oracle")
        for d in big + small:
            d.free()
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 1)
    assert ctx.check_device_error() == 0


def test_noalloc_refuses_batches_beyond_the_scratch_size(ctx):
    """5,000 sequences on the stream-K schedule need (512 + 5000) partial slots of
    14 x 66 floats, about 20 MB, more than TMAC_SCRATCH_BYTES (16 MiB): refused
    before any launch, and the output is untouched."""
    ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 2)
    try:
        n = 5000
        lens = np.full(n, 16, np.int32)
        offs = np.arange(n, dtype=np.int64) * 16
        dev = [ctx.upload(a) for a in (np.zeros((n, QD), np.float32), np.zeros((n * 16, KVD), np.float32),
                                       np.zeros((n * 16, KVD), np.float32), offs, lens)]
        dev += [ctx.empty((n, QD)), ctx.empty((1, QD))]
        dev[5].fill_bytes(0x7F)
        rc = call_noalloc(ctx, dev, n, 16, n * 16)
        assert rc == tmac_attn.TMAC_ERR_CAPACITY, rc
        assert "scratch" in ctx.lib.tmac_last_error(ctx.handle).decode()
        assert np.all(dev[5].numpy().view(np.uint32) == 0x7F7F7F7F)
        for d in dev:
            d.free()
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 1)
