"""Several contexts used at the same time from several host threads.

A serving process may hold one context per engine and drive them from
separate threads (the contract: one context is used from one host thread at a
time; different contexts are independent).  Each context owns its module,
workspace, RoPE tables, position-counter row caches and graphs, so calls on
different contexts must not disturb each other even while their kernels run
concurrently on the one GPU, and no call may end another thread's step
capture: on this runtime a legacy-stream copy or a device-wide synchronize,
issued from any thread while a stream captures, fails and ends that capture,
so the library makes its own copies on a per-context stream and synchronizes
the device only while no capture is in progress (the threads here copy on
their own streams for the same reason).  Here three threads, each with its own context and
stream, loop over work that uses every per-context resource (a ragged decode
forced onto many splits, so through the split workspace and the combine
launch; a chunked prefill, whose tiles live in the workspace; a captured
4-layer step replayed at successive positions of a device-side counter, with
the RoPE row cache) on inputs seeded per thread, and check every result
against the oracle.  ctypes releases the GIL around each library call, so the
host side of the calls overlaps too.
"""
import threading

import numpy as np
import pytest

import oracle
import tmac_attn
from conftest import assert_close

pytestmark = pytest.mark.gpu
NH, NKV, HD = 14, 2, 64
QD, KVD = NH * HD, NKV * HD
N_THREADS, ITERS = 3, 4


def upload(ctx, s, host):
    """A device copy of host, copied on stream s (not on the legacy stream, whose
    operations would end a capture in progress in another thread)."""
    host = np.ascontiguousarray(host)
    d = ctx.empty(host.shape, host.dtype)
    d.copy_from(host, stream=s)
    return d


def worker(tid: int, errors: list) -> None:
    try:
        with tmac_attn.Context(0) as ctx:
            s = ctx.stream()
            up = lambda host: upload(ctx, s, host)  # noqa: E731
            base = 20000 + 100 * tid
            # ragged decode, 256-row splits (a different length set per thread)
            rng = np.random.default_rng(base)
            lens = rng.integers(1, 3000, 6).astype(np.int32)
            offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
            k = oracle.normal(base + 1, (int(lens.sum()), KVD))
            v = oracle.normal(base + 2, (int(lens.sum()), KVD))
            dk, dv, doff, dlen = up(k), up(v), up(offs), up(lens)
            dq, dout = ctx.empty((lens.size, QD)), ctx.empty((lens.size, QD))
            ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 256)
            # prefill: 2 sequences x 48 queries after 200 rows
            n_q, prefix = 48, 200
            cap = prefix + n_q
            pq = oracle.normal(base + 3, (2, n_q, QD))
            pk = oracle.normal(base + 4, (2 * cap, KVD))
            pv = oracle.normal(base + 5, (2 * cap, KVD))
            bf = lambda x: (((x.view(np.uint32).astype(np.uint64) + 0x7FFF  # noqa: E731
                              + ((x.view(np.uint32) >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)
            pq, pk, pv = bf(pq), bf(pk), bf(pv)
            dpq, dpk, dpv, dpo = up(pq), up(pk), up(pv), ctx.empty((2, n_q, QD))
            pref = oracle.prefill(pq, pk, pv, 2, n_q, prefix, cap, NH, NKV, HD)
            # captured 4-layer step over a device-side position counter
            L, lcap = 4, 64
            kc, vc = up(np.zeros((L, lcap, KVD), np.float32)), up(np.zeros((L, lcap, KVD), np.float32))
            lq, lk, lv = ctx.empty((L, QD)), ctx.empty((L, KVD)), ctx.empty((L, KVD))
            lo = ctx.empty((L, QD))
            pos = up(np.zeros(1, np.int32))
            ctx.rope_prepare(HD, 1e6, lcap)
            ctx.step_begin(s)
            for l in range(L):
                ctx.layer_attention_devpos(lq.at(l * QD), lk.at(l * KVD), lv.at(l * KVD), kc.at(l * lcap * KVD),
                                           vc.at(l * lcap * KVD), lo.at(l * QD), NH, NKV, HD, pos, lcap, 1e6, stream=s)
            ctx.pos_update(pos, 1, add=True, stream=s)
            g = ctx.step_end(s)
            ref_k = np.zeros((L, lcap, KVD), np.float32)
            ref_v = np.zeros((L, lcap, KVD), np.float32)
            try:
                for it in range(ITERS):
                    q = oracle.normal(base + 10 + it, (lens.size, QD))
                    dq.copy_from(q, stream=s)
                    ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, lens.size, NH, NKV, HD, 3000, stream=s)
                    ref = oracle.attention_ragged(q, k, v, offs, lens, NH, NKV, HD, n_threads=2)
                    assert_close(dout.numpy(stream=s), ref, f"thread {tid} ragged iteration {it}")
                    dpo.fill_bytes(0xFF, stream=s)
                    ctx.prefill(dpq, dpk, dpv, dpo, 2, n_q, prefix, cap, NH, NKV, HD, stream=s)
                    assert_close(dpo.numpy(stream=s), pref, f"thread {tid} prefill iteration {it}")
                    for step in range(2):  # two positions per iteration
                        p = 2 * it + step
                        xq = oracle.normal(base + 50 + p, (L, QD))
                        xk = oracle.normal(base + 51 + p, (L, KVD))
                        xv = oracle.normal(base + 52 + p, (L, KVD))
                        lq.copy_from(xq, stream=s)
                        lk.copy_from(xk, stream=s)
                        lv.copy_from(xv, stream=s)
                        ctx.graph_launch(g, s)
                        got = lo.numpy(stream=s)
                        for l in range(L):
                            out, _, _ = oracle.layer_step(xq[l], xk[l], xv[l], ref_k[l], ref_v[l], NH, NKV, HD, p, 1e6)
                            assert_close(got[l], out, f"thread {tid} layer {l} position {p}")
                assert int(pos.numpy(stream=s)[0]) == 2 * ITERS
                assert ctx.check_device_error() == 0
            finally:
                ctx.graph_destroy(g)
                ctx.destroy_stream(s)
    except BaseException as e:  # reported by the main thread
        errors.append((tid, repr(e)))


def test_contexts_in_parallel_threads():
    errors: list = []
    threads = [threading.Thread(target=worker, args=(t, errors)) for t in range(N_THREADS)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
