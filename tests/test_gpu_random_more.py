"""More seeded random sweeps over entry points, shapes, cache types and options.

Like tests/test_gpu_random_shapes.py, each case draws every parameter at once
and checks the result against the oracle (tmac_gguf.cpp:1093-1128 for the
attention, 990-1016 for RoPE): the batched decode with padded sequence strides,
the reference's attention_op on compiled and any-shape geometries, the four
chunked-prefill entry points (fp32 cache, narrow cache, paged cache, persistent
tile copy), and the stream-K schedule with a random number of workgroups.
Tolerance |gpu - ref| <= 2e-5 + 1e-4 |ref|.
"""
import numpy as np
import pytest

import oracle
import tmac_attn
from conftest import assert_close
from test_gpu_random_shapes import DTYPES, PR, SHAPES, paged_pool, store, widen

pytestmark = pytest.mark.gpu
HD = 64


def bf16_round(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


class Dev:
    """Device buffers of one case, freed together."""

    def __init__(self, ctx):
        self.ctx, self.bufs = ctx, []

    def up(self, x):
        d = self.ctx.upload(np.ascontiguousarray(x))
        self.bufs.append(d)
        return d

    def empty(self, shape, dtype=np.float32):
        d = self.ctx.empty(shape, dtype)
        self.bufs.append(d)
        return d

    def free(self):
        for d in self.bufs:
            d.free()


def set_options(ctx, **opts):
    names = {"kernel": tmac_attn.TMAC_OPT_KERNEL, "mfma": tmac_attn.TMAC_OPT_MFMA_DECODE,
             "split": tmac_attn.TMAC_OPT_SPLIT_LEN, "stream_k": tmac_attn.TMAC_OPT_STREAM_K,
             "groups": tmac_attn.TMAC_OPT_TARGET_GROUPS}
    for k, v in opts.items():
        ctx.set_option(names[k], v)


def reset_options(ctx):
    set_options(ctx, kernel=0, mfma=1, split=0, stream_k=1, groups=0)


@pytest.mark.parametrize("seed", range(32))
def test_random_batched_decode(ctx, seed):
    """decode_batched: n_seq sequences of n_pos rows at a padded stride."""
    rng = np.random.default_rng(9000 + seed)
    g, kv = SHAPES[int(rng.integers(len(SHAPES)))]
    dt = DTYPES[int(rng.integers(len(DTYPES)))]
    nh, kvd = g * kv, kv * HD
    n_seq = int(rng.integers(1, 9))
    n_pos = int(rng.choice([1, 2, 15, 16, 17, int(rng.integers(18, 3000))]))
    stride = n_pos + int(rng.integers(0, 20))
    opts = dict(kernel=int(rng.integers(0, 4)), mfma=int(rng.integers(0, 2)), split=int(rng.choice([0, 0, 32, 100])))
    what = f"seed {seed}: g={g} kv={kv} dt={dt} n_seq={n_seq} n_pos={n_pos} stride={stride} {opts}"
    d = Dev(ctx)
    try:
        q = oracle.normal(9100 + seed, (n_seq, nh * HD))
        rows = oracle.normal(9200 + seed, (n_seq * stride, kvd))
        vrows = oracle.normal(9300 + seed, (n_seq * stride, kvd))
        kb, vb = store(rows, dt, kv), store(vrows, dt, kv)
        out = d.empty((n_seq, nh * HD))
        set_options(ctx, **opts)
        ctx.decode_batched(d.up(q), d.up(kb), d.up(vb), out, n_seq, nh, kv, HD, n_pos, stride, kv_dtype=dt)
        offs = np.arange(n_seq, dtype=np.int64) * stride
        ref = oracle.attention_ragged(q, widen(kb, dt, kv), widen(vb, dt, kv), offs, np.full(n_seq, n_pos, np.int32),
                                      nh, kv, HD, n_threads=8)
        assert_close(out.numpy(), ref, what)
        assert ctx.check_device_error() == 0, what
    finally:
        reset_options(ctx)
        d.free()


@pytest.mark.parametrize("seed", range(32))
def test_random_attention_op(ctx, seed):
    """The reference's attention_op: rows 0..past_len of a cache with spare
    capacity, compiled GQA shapes at head_dim 64 and any-shape geometries
    (any group, any even head_dim up to 256) on the fp32 path."""
    rng = np.random.default_rng(9400 + seed)
    if seed % 2:
        g, kv = SHAPES[int(rng.integers(len(SHAPES)))]
        hd = HD
    else:
        kv = int(rng.integers(1, 5))
        g = int(rng.integers(1, 10))
        hd = int(rng.choice([2, 32, 64, 66, 96, 128, 200, 256]))
    nh = g * kv
    past = int(rng.choice([0, 1, 15, 16, int(rng.integers(17, 2000))]))
    cap = past + 1 + int(rng.integers(0, 10))
    opts = dict(kernel=int(rng.integers(0, 4)), split=int(rng.choice([0, 0, 32])))
    what = f"seed {seed}: nh={nh} kv={kv} hd={hd} past={past} {opts}"
    d = Dev(ctx)
    try:
        q = oracle.normal(9500 + seed, nh * hd)
        k = oracle.normal(9501 + seed, (cap, kv * hd))
        v = oracle.normal(9502 + seed, (cap, kv * hd))
        out = d.empty(nh * hd)
        set_options(ctx, **opts)
        ctx.attention_op(d.up(q), d.up(k), d.up(v), out, nh, kv, hd, past)
        ref = oracle.attention(q, k, v, nh, kv, hd, past)
        assert_close(out.numpy(), ref, what)
    finally:
        reset_options(ctx)
        d.free()


@pytest.mark.parametrize("seed", range(32))
def test_random_prefill(ctx, seed):
    """Chunked prefill through one of its four entry points on random shapes,
    lengths and cache types.  The kernel's MFMA operands are bf16: the cache
    rows are widened exactly and rounded to bf16 (nearest even), so the
    reference is the oracle on those rows and on the bf16-rounded queries."""
    rng = np.random.default_rng(9600 + seed)
    g, kv = SHAPES[int(rng.integers(len(SHAPES)))]
    nh, kvd = g * kv, kv * HD
    entry = ["prefill", "prefill_kv", "prefill_paged", "tiles"][seed % 4]
    dt = tmac_attn.TMAC_KV_F32 if entry in ("prefill", "tiles") else DTYPES[int(rng.integers(len(DTYPES)))]
    n_seq = int(rng.integers(1, 4))
    n_q = int(rng.choice([1, 15, 16, 17, int(rng.integers(2, 150))]))
    prefix = int(rng.choice([0, int(rng.integers(1, 80)), int(rng.integers(80, 600))]))
    cap = prefix + n_q + int(rng.integers(0, 20))
    what = f"seed {seed}: {entry} g={g} kv={kv} dt={dt} n_seq={n_seq} n_q={n_q} prefix={prefix} cap={cap}"
    d = Dev(ctx)
    try:
        q = bf16_round(oracle.normal(9700 + seed, (n_seq, n_q, nh * HD)))
        k = oracle.normal(9701 + seed, (n_seq, cap, kvd))
        v = oracle.normal(9702 + seed, (n_seq, cap, kvd))
        kb = store(k.reshape(-1, kvd), dt, kv).reshape(n_seq, cap, -1)
        vb = store(v.reshape(-1, kvd), dt, kv).reshape(n_seq, cap, -1)
        kw = bf16_round(widen(kb.reshape(n_seq * cap, -1), dt, kv)).reshape(n_seq, cap, kvd)
        vw = bf16_round(widen(vb.reshape(n_seq * cap, -1), dt, kv)).reshape(n_seq, cap, kvd)
        out = d.empty((n_seq, n_q, nh * HD))
        dq = d.up(q)
        if entry == "prefill":
            ctx.prefill(dq, d.up(kb), d.up(vb), out, n_seq, n_q, prefix, cap, nh, kv, HD)
        elif entry == "prefill_kv":
            ctx.prefill(dq, d.up(kb), d.up(vb), out, n_seq, n_q, prefix, cap, nh, kv, HD, kv_dtype=dt)
        elif entry == "prefill_paged":
            used = prefix + n_q
            k_st = [kb[s, :used] for s in range(n_seq)]
            v_st = [vb[s, :used] for s in range(n_seq)]
            n_pages = n_seq * ((used + PR - 1) // PR) + 3
            kp, table = paged_pool(k_st, n_pages, np.random.default_rng(9800 + seed))
            vp, _ = paged_pool(v_st, n_pages, np.random.default_rng(9800 + seed))
            ctx.prefill_paged(dq, d.up(kp), d.up(vp), n_pages, d.up(table), table.shape[1], out, n_seq, n_q, prefix,
                              nh, kv, HD, kv_dtype=dt)
        else:
            tiles = d.empty(ctx.prefill_tiles_bytes(n_seq, kv, cap), np.uint8)
            dk, dv = d.up(kb), d.up(vb)
            # pack the prefix first, then the chunk's rows, as a chunked prompt does
            if prefix:
                ctx.prefill_pack_rows(dk, dv, cap, tiles, cap, n_seq, kv, HD, 0, prefix)
            ctx.prefill_pack_rows(dk, dv, cap, tiles, cap, n_seq, kv, HD, prefix, prefix + n_q)
            ctx.prefill_tiles(dq, tiles, cap, out, n_seq, n_q, prefix, nh, kv, HD)
        ref = oracle.prefill(q, kw.reshape(-1, kvd), vw.reshape(-1, kvd), n_seq, n_q, prefix, cap, nh, kv, HD,
                             n_threads=8)
        assert_close(out.numpy(), ref, what)
        assert ctx.check_device_error() == 0, what
    finally:
        d.free()


@pytest.mark.parametrize("seed", range(32))
def test_random_stream_k(ctx, seed):
    """The stream-K schedule forced on ragged or paged batches with a random
    number of workgroups (1 .. 600, or one per CU), random shapes and caches."""
    rng = np.random.default_rng(9900 + seed)
    g, kv = SHAPES[int(rng.integers(len(SHAPES)))]
    dt = DTYPES[int(rng.integers(len(DTYPES)))]
    nh, kvd = g * kv, kv * HD
    paged = bool(seed % 2)
    n_seq = int(rng.integers(1, 40))
    lens = rng.integers(0, 1200, n_seq).astype(np.int32)
    lens[rng.random(n_seq) < 0.15] = 0
    if lens.max() == 0:
        lens[0] = 1
    groups = int(rng.choice([1, 2, 7, 37, 600, 0]))
    what = f"seed {seed}: g={g} kv={kv} dt={dt} paged={paged} n_seq={n_seq} groups={groups}"
    d = Dev(ctx)
    try:
        q = oracle.normal(9910 + seed, (n_seq, nh * HD))
        k_st = [store(oracle.normal(9920 + 50 * seed + s, (max(int(l), 1), kvd)), dt, kv)[:l] for s, l in
                enumerate(lens)]
        v_st = [store(oracle.normal(9921 + 50 * seed + s, (max(int(l), 1), kvd)), dt, kv)[:l] for s, l in
                enumerate(lens)]
        out = d.empty((n_seq, nh * HD))
        set_options(ctx, stream_k=2, groups=groups)
        if paged:
            n_pages = int(sum((l + PR - 1) // PR for l in lens)) + 3
            kp, table = paged_pool([r if r.shape[0] else r[:0] for r in k_st], n_pages,
                                   np.random.default_rng(9930 + seed))
            vp, _ = paged_pool([r if r.shape[0] else r[:0] for r in v_st], n_pages, np.random.default_rng(9930 + seed))
            ctx.decode_paged(d.up(q), d.up(kp), d.up(vp), n_pages, d.up(table), table.shape[1], d.up(lens), out,
                             n_seq, nh, kv, HD, int(lens.max()), kv_dtype=dt)
        else:
            offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
            kcat = np.concatenate([r for r in k_st if r.shape[0]])
            vcat = np.concatenate([r for r in v_st if r.shape[0]])
            ctx.decode_ragged(d.up(q), d.up(kcat), d.up(vcat), d.up(offs), d.up(lens), out, n_seq, nh, kv, HD,
                              int(lens.max()), kv_dtype=dt)
        got = out.numpy()
        nz = lens > 0
        assert np.all(got[~nz] == 0), what
        offs_nz = np.concatenate([[0], np.cumsum(lens[nz][:-1])]).astype(np.int64)
        ref = oracle.attention_ragged(q[nz], np.concatenate([widen(r, dt, kv) for r in k_st if r.shape[0]]),
                                      np.concatenate([widen(r, dt, kv) for r in v_st if r.shape[0]]), offs_nz,
                                      lens[nz], nh, kv, HD, n_threads=8)
        assert_close(got[nz], ref, what)
        assert ctx.check_device_error() == 0, what
    finally:
        reset_options(ctx)
        d.free()
