"""GPU tests of the RoPE row cache of device-side position counters.

A fused layer step reading its position from device memory (tmac_layer_attention_devpos)
takes the RoPE row of that position from the counter's two-slot row cache when a slot is
tagged with (position, RoPE table), and from the table otherwise; tmac_pos_update writes the
row of the position it sets into the cache.  These tests drive the paths a graph sweep does
not: positions that jump, positions copied into the counter without tmac_pos_update (no slot
matches), two counters sharing one table, one counter alternating between two tables (RoPE
bases), and more counters than the context has row caches.  Every output is checked
against the oracle's layer step (tmac_gguf.cpp:990-1016, 1090-1128) and the caches bit for
bit."""
import numpy as np
import pytest

import oracle
from conftest import assert_close

pytestmark = pytest.mark.gpu
NH, NKV, HD = 14, 2, 64
QD, KVD = NH * HD, NKV * HD


class Seq:
    """One sequence's layer cache on the GPU and in the oracle, with its own position counter."""

    def __init__(self, ctx, cap, seed):
        self.ctx, self.cap, self.seed = ctx, cap, seed
        self.kc = ctx.upload(np.zeros((cap, KVD), np.float32))
        self.vc = ctx.upload(np.zeros((cap, KVD), np.float32))
        self.ref_k = np.zeros((cap, KVD), np.float32)
        self.ref_v = np.zeros((cap, KVD), np.float32)
        self.pos = ctx.upload(np.zeros(1, np.int32))
        self.dq, self.dkn, self.dvn, self.dout = ctx.empty(QD), ctx.empty(KVD), ctx.empty(KVD), ctx.empty(QD)

    def step(self, p, base, what, direct=False):
        q = oracle.normal(self.seed * 1000 + p, QD)
        kn = oracle.normal(self.seed * 1000 + p + 500, KVD)
        vn = oracle.normal(self.seed * 1000 + p + 700, KVD)
        self.dq.copy_from(q)
        self.dkn.copy_from(kn)
        self.dvn.copy_from(vn)
        if direct:  # the counter written by a copy: its row cache is not refreshed
            self.pos.copy_from(np.array([p], np.int32))
        else:
            self.ctx.pos_update(self.pos, p)
        self.ctx.layer_attention_devpos(self.dq, self.dkn, self.dvn, self.kc, self.vc, self.dout, NH, NKV, HD,
                                        self.pos, self.cap, base)
        self.ctx.synchronize(None)
        ref, _, _ = oracle.layer_step(q, kn, vn, self.ref_k, self.ref_v, NH, NKV, HD, p, base)
        assert_close(self.dout.numpy(), ref, what)

    def check_caches(self):
        np.testing.assert_array_equal(self.kc.numpy(), self.ref_k)
        np.testing.assert_array_equal(self.vc.numpy(), self.ref_v)

    def free(self):
        for d in (self.kc, self.vc, self.pos, self.dq, self.dkn, self.dvn, self.dout):
            d.free()


def test_positions_that_jump(ctx):
    """Positions set through tmac_pos_update in any order (forward, backward,
    the same twice) find their row in the cache; positions written into the
    counter by a plain copy find a slot tagged with an older position, and the
    row is read from the table."""
    s = Seq(ctx, 256, 31)
    try:
        for p in (0, 1, 2, 40, 41, 7, 8, 8, 200, 255, 3):
            s.step(p, 1e6, f"position {p}")
        for p in (9, 10, 11, 100, 4):
            s.step(p, 1e6, f"position {p} (copied into the counter)", direct=True)
        s.check_caches()
    finally:
        s.free()
    assert ctx.check_device_error() == 0


def test_two_counters_share_a_table(ctx):
    """Two sequences at different positions, interleaved step by step on the
    same RoPE table: each counter's row cache holds its own rows."""
    a, b = Seq(ctx, 256, 41), Seq(ctx, 256, 42)
    try:
        for i in range(6):
            a.step(10 + i, 1e6, f"sequence a position {10 + i}")
            b.step(200 + i, 1e6, f"sequence b position {200 + i}")
        a.check_caches()
        b.check_caches()
    finally:
        a.free()
        b.free()
    assert ctx.check_device_error() == 0


def test_one_counter_two_tables(ctx):
    """One counter alternating between RoPE bases 1e6 and 1e4 (two tables): a
    slot written from one table never serves the other."""
    s1, s2 = Seq(ctx, 128, 51), Seq(ctx, 128, 52)
    s2.pos.free()
    s2.pos = s1.pos  # the same device counter
    try:
        for p in range(5):
            s1.step(p, 1e6, f"base 1e6 position {p}")
            s2.step(p, 1e4, f"base 1e4 position {p}")
        s1.check_caches()
        s2.check_caches()
    finally:
        s2.pos = None
        for d in (s2.kc, s2.vc, s2.dq, s2.dkn, s2.dvn, s2.dout):
            d.free()
        s1.free()
    assert ctx.check_device_error() == 0


def test_more_counters_than_row_caches(ctx):
    """Counters beyond the context's row caches run without one (the RoPE row
    is read after the position) and give the same results."""
    seqs = [Seq(ctx, 64, 60 + i) for i in range(70)]
    try:
        for i, s in enumerate(seqs):
            for p in (0, 1, 2):
                s.step(p, 1e6, f"counter {i} position {p}")
            s.check_caches()
    finally:
        for s in seqs:
            s.free()
    assert ctx.check_device_error() == 0
