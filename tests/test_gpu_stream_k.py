"""GPU parity of the stream-K ragged decode (fp32 caches; one of the two
schedules of tmac_attention_decode_ragged, forced here with TMAC_OPT_STREAM_K=2).

The batch's rows, each sequence padded to 16 rows, are cut on the device into
equal ranges, one workgroup each; a sequence may span several ranges and a
range several sequences.  The workgroup count is swept from 1 (one workgroup
takes the whole batch) to more than the rows allow (64-row ranges, a 5,000-row
sequence over 79 of them), and the row-count hint (unused by this schedule)
from none to far too low.  Every result is checked against the
oracle (tmac_gguf.cpp:1093-1128 per sequence) with the attention tolerance
2e-5 + 1e-4 |ref|, and empty and over-long sequences keep the entry point's
contract (zeros; NaN and error bit 1).
"""
import numpy as np
import pytest

import oracle
import tmac_attn
from conftest import assert_close
from test_gpu_kv_q8_paged import build_pool, data, store, widen

pytestmark = pytest.mark.gpu

NH, NKV, HD = 14, 2, 64
KVD = NKV * HD
PR = tmac_attn.PAGE_ROWS


@pytest.fixture(autouse=True)
def stream_k(ctx):
    ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 2)
    yield
    ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 1)


def ragged_batch(ctx, seed, lens):
    lens = np.asarray(lens, np.int32)
    offs = np.concatenate([[0], np.cumsum(lens[:-1], dtype=np.int64)]).astype(np.int64)
    total = int(lens.sum())
    k, v = oracle.normal(seed, (max(total, 1), KVD)), oracle.normal(seed + 1, (max(total, 1), KVD))
    q = oracle.normal(seed + 2, (lens.size, NH * HD))
    return lens, offs, total, k, v, q


def reference(q, k, v, offs, lens):
    ref = np.zeros((lens.size, NH * HD), np.float32)
    nz = lens > 0
    ref[nz] = oracle.attention_ragged(q[nz], k, v, offs[nz], lens[nz], NH, NKV, HD, n_threads=8)
    return ref


@pytest.mark.parametrize("groups", [1, 3, 37, 0, 600])
def test_stream_k_matches_oracle(ctx, groups):
    lens, offs, total, k, v, q = ragged_batch(
        ctx, 4100, [0, 1, 15, 16, 17, 63, 64, 65, 300, 2048, 5000, 0, 33, 7, 4097, 1])
    ref = reference(q, k, v, offs, lens)
    dq, dk, dv, doff, dlen = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.upload(offs), ctx.upload(lens)
    dout = ctx.empty((lens.size, NH * HD))
    ctx.set_option(tmac_attn.TMAC_OPT_TARGET_GROUPS, groups)
    try:
        for hint in (0, 1, total // 3, total):
            dout.fill_bytes(0xFF)
            ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, lens.size, NH, NKV, HD, int(lens.max()),
                              total_rows=hint)
            assert_close(dout.numpy(), ref, f"stream-K groups={groups} hint={hint}")
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_TARGET_GROUPS, 0)
    assert ctx.check_device_error() == 0


def test_stream_k_equals_unit_grid(ctx):
    """Both schedules of the fp32 ragged decode on 200 sequences of 1..3000 rows
    agree with the oracle (the merge order differs, so not bit for bit)."""
    rng = np.random.default_rng(41)
    lens, offs, total, k, v, q = ragged_batch(ctx, 4200, rng.integers(1, 3001, 200))
    ref = reference(q, k, v, offs, lens)
    dq, dk, dv, doff, dlen = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.upload(offs), ctx.upload(lens)
    dout = ctx.empty((lens.size, NH * HD))
    try:
        for sk in (2, 0):
            ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, sk)
            dout.fill_bytes(0xFF)
            ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, lens.size, NH, NKV, HD, int(lens.max()),
                              total_rows=total)
            assert_close(dout.numpy(), ref, f"stream_k={sk}")
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 2)
    assert ctx.check_device_error() == 0


def test_stream_k_over_long_sequence(ctx):
    """A length above max_len gives a NaN output and error bit 1; the other
    sequences of the batch, before and after it in the row space, are exact."""
    lens, offs, total, k, v, q = ragged_batch(ctx, 4300, [700, 900, 1200, 5])
    ref = reference(q, k, v, offs, lens)
    dq, dk, dv, doff, dlen = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.upload(offs), ctx.upload(lens)
    dout = ctx.empty((lens.size, NH * HD))
    ctx.set_option(tmac_attn.TMAC_OPT_TARGET_GROUPS, 9)
    try:
        ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, lens.size, NH, NKV, HD, 1000, total_rows=total)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_TARGET_GROUPS, 0)
    got = dout.numpy()
    assert np.all(np.isnan(got[2]))
    keep = np.array([0, 1, 3])
    assert_close(got[keep], ref[keep], "sequences beside the over-long one")
    assert ctx.check_device_error() == tmac_attn.TMAC_ERR_DEVICE_FAULT
    assert ctx.check_device_error() == 0


def test_stream_k_graph_replay_new_lengths(ctx):
    """A captured stream-K decode reads the lengths on the device: replays after
    the lengths (and queries) change, within the captured max_len and row-count
    hint, are exact, with eager calls of other shapes between the replays."""
    max_len, n_seq, cap = 4000, 24, 24 * 4000
    k, v = oracle.normal(4400, (cap, KVD)), oracle.normal(4401, (cap, KVD))
    offs = np.arange(n_seq, dtype=np.int64) * max_len
    dk, dv, doff = ctx.upload(k), ctx.upload(v), ctx.upload(offs)
    dq, dlen, dout = ctx.empty((n_seq, NH * HD)), ctx.empty(n_seq, np.int32), ctx.empty((n_seq, NH * HD))
    s = ctx.stream()
    rng = np.random.default_rng(44)
    hint = n_seq * max_len // 2
    try:
        dlen.copy_from(np.full(n_seq, 1, np.int32))
        ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, n_seq, NH, NKV, HD, max_len, total_rows=hint, stream=s)
        ctx.synchronize(s)
        ctx.step_begin(s)
        ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, n_seq, NH, NKV, HD, max_len, total_rows=hint, stream=s)
        g = ctx.step_end(s)
        try:
            for rep in range(4):
                lens = rng.integers(0, max_len + 1, n_seq).astype(np.int32)
                q = oracle.normal(4500 + rep, (n_seq, NH * HD))
                dq.copy_from(q)
                dlen.copy_from(lens)
                ctx.graph_launch(g, s)
                ctx.synchronize(s)
                assert_close(dout.numpy(), reference(q, k, v, offs, lens), f"replay {rep}")
                e_lens = np.full(3, 2500, np.int32)  # an eager call of another shape in between
                ctx.decode_ragged(dq, dk, dv, doff, ctx.upload(e_lens), dout, 3, NH, NKV, HD, 2500, stream=s)
                ctx.synchronize(s)
                assert_close(dout.numpy()[:3], reference(q[:3], k, v, offs[:3], e_lens), f"eager {rep}")
        finally:
            ctx.graph_destroy(g)
    finally:
        ctx.destroy_stream(s)
    assert ctx.check_device_error() == 0


def to_pages(k, v, offs, lens, rng, spare=5):
    """Scatters each sequence's rows over 16-row pages of a pool, in random
    pool order; returns (k pool, v pool, block table, pages in the pool)."""
    pr = tmac_attn.PAGE_ROWS
    need = [(int(n) + pr - 1) // pr for n in lens]
    n_pages = sum(need) + spare
    perm = rng.permutation(n_pages)
    table = np.zeros((lens.size, max(max(need), 1)), np.int32)
    kp = np.zeros((n_pages * pr,) + k.shape[1:], k.dtype)
    vp = np.zeros_like(kp)
    nxt = 0
    for s, n in enumerate(lens):
        for j in range(need[s]):
            pg = int(perm[nxt])
            nxt += 1
            table[s, j] = pg
            r = min(int(n) - j * pr, pr)
            kp[pg * pr:pg * pr + r] = k[offs[s] + j * pr:offs[s] + j * pr + r]
            vp[pg * pr:pg * pr + r] = v[offs[s] + j * pr:offs[s] + j * pr + r]
    return kp, vp, table, n_pages


@pytest.mark.parametrize("groups", [1, 37, 0])
def test_stream_k_paged_matches_oracle(ctx, groups):
    """The stream-K schedule over paged fp32 caches (pages in random pool
    order), against the oracle on the same rows."""
    lens, offs, total, k, v, q = ragged_batch(
        ctx, 4600, [0, 1, 15, 16, 17, 63, 64, 65, 300, 2048, 5000, 0, 33, 7, 4097, 1])
    ref = reference(q, k, v, offs, lens)
    kp, vp, table, n_pages = to_pages(k, v, offs, lens, np.random.default_rng(46))
    dq, dk, dv, dtab, dlen = ctx.upload(q), ctx.upload(kp), ctx.upload(vp), ctx.upload(table), ctx.upload(lens)
    dout = ctx.empty((lens.size, NH * HD))
    dout.fill_bytes(0xFF)
    ctx.set_option(tmac_attn.TMAC_OPT_TARGET_GROUPS, groups)
    try:
        ctx.decode_paged(dq, dk, dv, n_pages, dtab, table.shape[1], dlen, dout, lens.size, NH, NKV, HD,
                         int(lens.max()))
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_TARGET_GROUPS, 0)
    assert_close(dout.numpy(), ref, f"paged stream-K groups={groups}")
    assert ctx.check_device_error() == 0


def test_stream_k_paged_bad_page_is_reported(ctx):
    """A block-table entry outside the pool is clamped into it (every access
    stays in bounds) and sets error bit 2; sequences with valid tables are exact."""
    lens, offs, total, k, v, q = ragged_batch(ctx, 4700, [100, 40, 300])
    ref = reference(q, k, v, offs, lens)
    kp, vp, table, n_pages = to_pages(k, v, offs, lens, np.random.default_rng(47))
    table[1, 1] = n_pages + 3
    dq, dk, dv, dtab, dlen = ctx.upload(q), ctx.upload(kp), ctx.upload(vp), ctx.upload(table), ctx.upload(lens)
    dout = ctx.empty((lens.size, NH * HD))
    ctx.decode_paged(dq, dk, dv, n_pages, dtab, table.shape[1], dlen, dout, lens.size, NH, NKV, HD, 300)
    keep = np.array([0, 2])
    assert_close(dout.numpy()[keep], ref[keep], "sequences with valid block tables")
    assert ctx.check_device_error() == tmac_attn.TMAC_ERR_DEVICE_FAULT
    assert ctx.check_device_error() == 0


NARROW = [tmac_attn.TMAC_KV_BF16, tmac_attn.TMAC_KV_F16, tmac_attn.TMAC_KV_Q8_0]


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("dt", NARROW)
def test_stream_k_mfma_matches_oracle(ctx, dt, paged):
    """The stream-K schedule on the MFMA decode (bf16 / fp16 / Q8_0 caches),
    contiguous ragged and paged, for 1, 37 and one-per-CU workgroups, against
    the oracle over the cache's exactly widened rows.  Rows of very different
    magnitudes exercise the Q8_0 block scales."""
    lens = np.array([0, 1, 15, 16, 17, 63, 64, 65, 300, 2048, 5000, 0, 33, 7, 4097, 1], np.int32)
    offs = np.concatenate([[0], np.cumsum(lens[:-1], dtype=np.int64)]).astype(np.int64)
    total = int(lens.sum())
    kb = store(data(4800 + dt, (total, KVD), 3), dt)
    vb = store(data(4810 + dt, (total, KVD), 3), dt)
    q = data(4820 + dt, (lens.size, NH * HD))
    ref = reference(q, widen(kb, dt), widen(vb, dt), offs, lens)
    dq, dlen, dout = ctx.upload(q), ctx.upload(lens), ctx.empty((lens.size, NH * HD))
    if paged:
        kp, vp, table, n_pages = to_pages(kb, vb, offs, lens, np.random.default_rng(48))
        dk, dv, dtab = ctx.upload(kp), ctx.upload(vp), ctx.upload(table)
    else:
        dk, dv, doff = ctx.upload(kb), ctx.upload(vb), ctx.upload(offs)
    try:
        for groups in (1, 37, 0):
            ctx.set_option(tmac_attn.TMAC_OPT_TARGET_GROUPS, groups)
            dout.fill_bytes(0xFF)
            if paged:
                ctx.decode_paged(dq, dk, dv, n_pages, dtab, table.shape[1], dlen, dout, lens.size, NH, NKV, HD,
                                 int(lens.max()), kv_dtype=dt)
            else:
                ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, lens.size, NH, NKV, HD, int(lens.max()),
                                  kv_dtype=dt)
            assert_close(dout.numpy(), ref, f"MFMA stream-K dt={dt} paged={paged} groups={groups}")
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_TARGET_GROUPS, 0)
    assert ctx.check_device_error() == 0


def test_stream_k_single_long_sequence(ctx):
    """One 16,384-row sequence over every workgroup (64-row ranges: 256
    partials, merged by the combine in chunks of 32), then the same rows as
    two sequences split mid-range."""
    lens, offs, total, k, v, q = ragged_batch(ctx, 4900, [16384])
    ref = reference(q, k, v, offs, lens)
    dq, dk, dv, doff, dlen = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.upload(offs), ctx.upload(lens)
    dout = ctx.empty((1, NH * HD))
    ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, 1, NH, NKV, HD, 16384)
    assert_close(dout.numpy(), ref, "one sequence over all workgroups")
    lens2 = np.array([10001, 6383], np.int32)
    offs2 = np.array([0, 10001], np.int64)
    q2 = oracle.normal(4903, (2, NH * HD))
    dq2, dout2 = ctx.upload(q2), ctx.empty((2, NH * HD))
    ctx.decode_ragged(dq2, dk, dv, ctx.upload(offs2), ctx.upload(lens2), dout2, 2, NH, NKV, HD, 10001)
    assert_close(dout2.numpy(), reference(q2, k, v, offs2, lens2), "two sequences of the same rows")
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("paged", [False, True])
def test_stream_k_no_rows(ctx, paged):
    """Batches with no rows to attend: all sequences empty (zeros), then all
    longer than max_len (NaN and error bit 1).  No workgroup has a range;
    the combine writes every output."""
    k = oracle.normal(5000, (64, KVD))
    table = np.arange(4, dtype=np.int32).reshape(1, 4).repeat(3, 0)
    dk, dv, dtab = ctx.upload(k), ctx.upload(k), ctx.upload(table)
    doff = ctx.upload(np.zeros(3, np.int64))
    dq, dout = ctx.upload(oracle.normal(5001, (3, NH * HD))), ctx.empty((3, NH * HD))
    for lens, want_err in ((np.zeros(3, np.int32), 0), (np.full(3, 60, np.int32), tmac_attn.TMAC_ERR_DEVICE_FAULT)):
        dout.fill_bytes(0x3F)
        dlen = ctx.upload(lens)
        if paged:
            ctx.decode_paged(dq, dk, dv, 4, dtab, 4, dlen, dout, 3, NH, NKV, HD, 48)
        else:
            ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, 3, NH, NKV, HD, 48)
        got = dout.numpy()
        assert np.all(got == 0) if want_err == 0 else np.all(np.isnan(got))
        assert ctx.check_device_error() == want_err
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("groups", [1, 37, 0])
def test_stream_k_paged_layer_step(ctx, groups):
    """The batched paged layer step (fp32) on the stream-K schedule: sequences
    at positions from 0 to 2,999 (page boundaries among them) get RoPE, their
    new row written into its page and attention over rows 0..pos; the segment
    holding row pos takes the new token.  Outputs against the oracle, pools
    byte for byte."""
    f32 = tmac_attn.TMAC_KV_F32
    rng = np.random.default_rng(52 + groups)
    positions = rng.integers(0, 3000, 40).astype(np.int32)
    positions[:6] = [0, 1, 15, 16, 31, 2047]
    n_seq = positions.size
    max_len = int(positions.max()) + 1
    k_rows = [data(5100 + s, (int(p) + 1, KVD)) for s, p in enumerate(positions)]
    v_rows = [data(5200 + s, (int(p) + 1, KVD)) for s, p in enumerate(positions)]
    n_pages = int(sum((p + PR) // PR for p in positions)) + 5
    kp, table = build_pool(k_rows, f32, n_pages, np.random.default_rng(53))
    vp, _ = build_pool(v_rows, f32, n_pages, np.random.default_rng(53))
    q, kn, vn = data(5300, (n_seq, NH * HD)), data(5301, (n_seq, KVD)), data(5302, (n_seq, KVD))
    dq, dkn, dvn = ctx.upload(q), ctx.upload(kn), ctx.upload(vn)
    dk, dv, dtab, dpos = ctx.upload(kp), ctx.upload(vp), ctx.upload(table), ctx.upload(positions)
    dout = ctx.empty((n_seq, NH * HD))
    ctx.set_option(tmac_attn.TMAC_OPT_TARGET_GROUPS, groups)
    try:
        ctx.layer_attention_paged(dq, dkn, dvn, dk, dv, n_pages, dtab, table.shape[1], dpos, dout, n_seq, NH, NKV,
                                  HD, max_len, 1e6)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_TARGET_GROUPS, 0)
    got, kp_got, vp_got = dout.numpy(), dk.numpy(), dv.numpy()
    kp_ref, vp_ref = kp.copy(), vp.copy()
    for s, p in enumerate(positions):
        qr, kr = oracle.rope(q[s], kn[s], NH, NKV, HD, int(p), 1e6)
        row = table[s, p // PR] * PR + p % PR
        kp_ref[row] = kr
        vp_ref[row] = vn[s]
        rows = np.array([table[s, r // PR] * PR + r % PR for r in range(p + 1)])
        ref = oracle.attention(qr, kp_ref[rows], vp_ref[rows], NH, NKV, HD, int(p))
        assert_close(got[s], ref, f"stream-K paged layer groups={groups} seq {s} pos {p}")
    np.testing.assert_array_equal(kp_got, kp_ref)
    np.testing.assert_array_equal(vp_got, vp_ref)
    assert ctx.check_device_error() == 0


def test_stream_k_paged_layer_bad_position(ctx):
    """A position past the pages of the block table sets error bit 0 and leaves
    that sequence's output and the pools untouched; the others are exact."""
    positions = np.array([20, 40, 70], np.int32)
    k_rows = [data(5400 + s, (int(p) + 1, KVD)) for s, p in enumerate(positions)]
    kp, table = build_pool(k_rows, tmac_attn.TMAC_KV_F32, 12, np.random.default_rng(54))
    table = table[:, :3]  # 48 rows per sequence: position 70 is outside
    q, kn, vn = data(5500, (3, NH * HD)), data(5501, (3, KVD)), data(5502, (3, KVD))
    dq, dkn, dvn, dk, dtab = ctx.upload(q), ctx.upload(kn), ctx.upload(vn), ctx.upload(kp), ctx.upload(table)
    dpos, dout = ctx.upload(positions), ctx.upload(np.full((3, NH * HD), 7.0, np.float32))
    ctx.layer_attention_paged(dq, dkn, dvn, dk, dk, 12, dtab, 3, dpos, dout, 3, NH, NKV, HD, 48, 1e6)
    got = dout.numpy()
    assert np.all(got[2] == 7.0)
    assert ctx.check_device_error() == tmac_attn.TMAC_ERR_DEVICE_FAULT
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("paged", [False, True])
def test_stream_k_twenty_thousand_sequences(ctx, paged):
    """20,000 sequences of 0..12 rows: the row total and the range search run
    over 79 rounds of 256 lengths in every workgroup."""
    rng = np.random.default_rng(56)
    lens = rng.integers(0, 13, 20000).astype(np.int32)
    lens, offs, total, k, v, q = ragged_batch(ctx, 5600, lens)
    ref = reference(q, k, v, offs, lens)
    dq, dlen, dout = ctx.upload(q), ctx.upload(lens), ctx.empty((lens.size, NH * HD))
    if paged:
        kp, vp, table, n_pages = to_pages(k, v, offs, lens, rng)
        ctx.decode_paged(dq, ctx.upload(kp), ctx.upload(vp), n_pages, ctx.upload(table), table.shape[1], dlen, dout,
                         lens.size, NH, NKV, HD, 12)
    else:
        ctx.decode_ragged(dq, ctx.upload(k), ctx.upload(v), ctx.upload(offs), dlen, dout, lens.size, NH, NKV, HD, 12)
    assert_close(dout.numpy(), ref, f"20,000 sequences paged={paged}")
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("dt", [tmac_attn.TMAC_KV_BF16, tmac_attn.TMAC_KV_Q8_0])
def test_stream_k_mfma_graph_replay(ctx, dt):
    """A captured MFMA stream-K decode (bf16 / Q8_0 ragged) replayed after the
    device-side lengths and the queries change; every replay against the
    oracle over the cache's widened rows."""
    max_len, n_seq = 3000, 20
    kb = store(data(5700 + dt, (n_seq * max_len, KVD), 2), dt)
    vb = store(data(5710 + dt, (n_seq * max_len, KVD), 2), dt)
    kw, vw = widen(kb, dt), widen(vb, dt)
    offs = np.arange(n_seq, dtype=np.int64) * max_len
    dk, dv, doff = ctx.upload(kb), ctx.upload(vb), ctx.upload(offs)
    dq, dlen, dout = ctx.empty((n_seq, NH * HD)), ctx.empty(n_seq, np.int32), ctx.empty((n_seq, NH * HD))
    s = ctx.stream()
    rng = np.random.default_rng(57)
    try:
        dlen.copy_from(np.ones(n_seq, np.int32))
        ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, n_seq, NH, NKV, HD, max_len, stream=s, kv_dtype=dt)
        ctx.synchronize(s)
        ctx.step_begin(s)
        ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, n_seq, NH, NKV, HD, max_len, stream=s, kv_dtype=dt)
        g = ctx.step_end(s)
        try:
            for rep in range(3):
                lens = rng.integers(0, max_len + 1, n_seq).astype(np.int32)
                q = data(5720 + rep, (n_seq, NH * HD))
                dq.copy_from(q)
                dlen.copy_from(lens)
                ctx.graph_launch(g, s)
                ctx.synchronize(s)
                assert_close(dout.numpy(), reference(q, kw, vw, offs, lens), f"dt={dt} replay {rep}")
        finally:
            ctx.graph_destroy(g)
    finally:
        ctx.destroy_stream(s)
    assert ctx.check_device_error() == 0
