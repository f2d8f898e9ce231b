"""Seeded random cases across the compiled GQA shapes, cache types, entry
points and options.

The other random-case tests hold the Qwen2 shape (14 / 2 heads) fixed and vary
lengths and options, or vary the shape on one entry point.  Here every case
draws all of them at once: a compiled (query heads per kv head, kv heads)
shape, a cache type (fp32, bf16, fp16, Q8_0), an entry point (ragged decode,
paged decode, the fused layer step with the position by value or in a device
counter, the batched paged layer step) and the kernel options (kernel choice,
MFMA or VALU decode for narrow caches, a forced split length, the stream-K
schedule), so that combinations no hand-written case names are still checked
against the oracle (tmac_gguf.cpp:990-1016, 1090-1091, 1093-1128): outputs to
|gpu - ref| <= 2e-5 + 1e-4 |ref|, written cache rows bit for bit.
"""
import numpy as np
import pytest

import oracle
import tmac_attn
from conftest import assert_close

pytestmark = pytest.mark.gpu
HD = 64
PR = tmac_attn.PAGE_ROWS
SHAPES = [(7, 2), (1, 1), (1, 2), (2, 2), (4, 2), (4, 4), (8, 1)]
DTYPES = [tmac_attn.TMAC_KV_F32, tmac_attn.TMAC_KV_BF16, tmac_attn.TMAC_KV_F16, tmac_attn.TMAC_KV_Q8_0]
ENTRIES = ["ragged", "paged", "layer", "layer_devpos", "layer_paged"]


def store(x, dt, kv):
    """fp32 rows [n][kv * 64] -> the cache's stored rows."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, kv * HD)
    if dt == tmac_attn.TMAC_KV_F32:
        return x.copy()
    if dt == tmac_attn.TMAC_KV_F16:
        return x.astype(np.float16).view(np.uint16)
    if dt == tmac_attn.TMAC_KV_BF16:
        u = x.view(np.uint32).astype(np.uint64)
        return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)
    return oracle.q8_kv_rows(x).reshape(-1, kv * oracle.Q8_HEAD_BYTES)


def widen(rows, dt, kv):
    """Stored rows -> fp32 [n][kv * 64], exactly."""
    if dt == tmac_attn.TMAC_KV_F32:
        return np.asarray(rows, np.float32).reshape(-1, kv * HD)
    if dt == tmac_attn.TMAC_KV_F16:
        return np.ascontiguousarray(rows, np.uint16).view(np.float16).astype(np.float32).reshape(-1, kv * HD)
    if dt == tmac_attn.TMAC_KV_BF16:
        return (np.ascontiguousarray(rows, np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(-1, kv * HD)
    return oracle.q8_kv_widen(rows).reshape(-1, kv * HD)


def paged_pool(rows_per_seq, n_pages, rng):
    """Scatters each sequence's stored rows over 16-row pages in random pool order.
    Returns pool [n_pages * 16][row], table [n_seq][max_pages]."""
    width = rows_per_seq[0].shape[1]
    max_pages = max(1, max((r.shape[0] + PR - 1) // PR for r in rows_per_seq))
    pool = np.zeros((n_pages * PR, width), rows_per_seq[0].dtype)
    perm = rng.permutation(n_pages)
    table = np.zeros((len(rows_per_seq), max_pages), np.int32)
    nxt = 0
    for s, r in enumerate(rows_per_seq):
        for j in range((r.shape[0] + PR - 1) // PR):
            table[s, j] = perm[nxt]
            nxt += 1
            seg = r[j * PR:(j + 1) * PR]
            pool[table[s, j] * PR:table[s, j] * PR + seg.shape[0]] = seg
    return pool, table


def pool_rows(table, s, n):
    return np.array([table[s, r // PR] * PR + r % PR for r in range(n)], np.int64)


@pytest.mark.parametrize("seed", range(64))
def test_random_shape_entry_option(ctx, seed):
    rng = np.random.default_rng(7000 + seed)
    g, kv = SHAPES[int(rng.integers(len(SHAPES)))]
    dt = DTYPES[int(rng.integers(len(DTYPES)))]
    entry = ENTRIES[seed % len(ENTRIES)]
    nh, kvd = g * kv, kv * HD
    kernel = int(rng.choice([tmac_attn.TMAC_KERNEL_AUTO, tmac_attn.TMAC_KERNEL_GROUP, tmac_attn.TMAC_KERNEL_HEAD,
                             tmac_attn.TMAC_KERNEL_HEADV]))
    mfma = int(rng.integers(0, 2))
    split_len = int(rng.choice([0, 0, 32, 256]))
    stream_k = int(rng.choice([0, 1, 2]))
    base = float(rng.choice([1e4, 1e6]))
    what = (f"seed {seed}: g={g} kv={kv} dt={dt} entry={entry} kernel={kernel} mfma={mfma} split={split_len} "
            f"stream_k={stream_k}")
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, kernel)
    ctx.set_option(tmac_attn.TMAC_OPT_MFMA_DECODE, mfma)
    ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, split_len)
    ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, stream_k)
    dev = []

    def up(x):
        d = ctx.upload(x)
        dev.append(d)
        return d
    try:
        if entry in ("ragged", "paged"):
            n_seq = int(rng.integers(1, 6))
            lens = rng.integers(1, 2500, n_seq).astype(np.int32)
            lens[rng.random(n_seq) < 0.2] = int(rng.choice([1, 15, 16, 17, 64]))
            q = oracle.normal(7100 + seed, (n_seq, nh * HD))
            k_st = [store(oracle.normal(7200 + 10 * seed + s, (int(lens[s]), kvd)), dt, kv) for s in range(n_seq)]
            v_st = [store(oracle.normal(7300 + 10 * seed + s, (int(lens[s]), kvd)), dt, kv) for s in range(n_seq)]
            out = ctx.empty((n_seq, nh * HD))
            dev.append(out)
            max_len = int(lens.max())
            if entry == "ragged":
                offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
                ctx.decode_ragged(up(q), up(np.concatenate(k_st)), up(np.concatenate(v_st)), up(offs), up(lens), out,
                                  n_seq, nh, kv, HD, max_len, int(lens.sum()) if rng.random() < 0.5 else 0,
                                  kv_dtype=dt)
            else:
                n_pages = int(sum((l + PR - 1) // PR for l in lens)) + 4
                prng = np.random.default_rng(7400 + seed)
                kp, table = paged_pool(k_st, n_pages, prng)
                vp, _ = paged_pool(v_st, n_pages, np.random.default_rng(7400 + seed))
                ctx.decode_paged(up(q), up(kp), up(vp), n_pages, up(table), table.shape[1], up(lens), out, n_seq, nh,
                                 kv, HD, max_len, kv_dtype=dt)
            offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
            ref = oracle.attention_ragged(q, np.concatenate([widen(r, dt, kv) for r in k_st]),
                                          np.concatenate([widen(r, dt, kv) for r in v_st]), offs, lens, nh, kv, HD,
                                          n_threads=8)
            assert_close(out.numpy(), ref, what)
        elif entry in ("layer", "layer_devpos"):
            pos = int(rng.choice([0, int(rng.integers(1, 80)), int(rng.integers(80, 3000))]))
            cap = pos + int(rng.integers(1, 30))
            q, kn, vn = oracle.normal(7500 + seed, nh * HD), oracle.normal(7501 + seed, kvd), \
                oracle.normal(7502 + seed, kvd)
            kb = store(oracle.normal(7503 + seed, (cap, kvd)), dt, kv)
            vb = store(oracle.normal(7504 + seed, (cap, kvd)), dt, kv)
            dk, dv, out = up(kb), up(vb), ctx.empty(nh * HD)
            dev.append(out)
            if entry == "layer":
                ctx.layer_attention(up(q), up(kn), up(vn), dk, dv, out, nh, kv, HD, pos, cap, base, kv_dtype=dt)
            else:
                ctx.layer_attention_devpos(up(q), up(kn), up(vn), dk, dv, out, nh, kv, HD,
                                           up(np.array([pos], np.int32)), cap, base, kv_dtype=dt)
            qr, kr = oracle.rope(q, kn, nh, kv, HD, pos, base)
            kb_ref, vb_ref = kb.copy(), vb.copy()
            kb_ref[pos] = store(kr, dt, kv)[0]
            vb_ref[pos] = store(vn, dt, kv)[0]
            np.testing.assert_array_equal(dk.numpy(), kb_ref, err_msg=what)
            np.testing.assert_array_equal(dv.numpy(), vb_ref, err_msg=what)
            ref = oracle.attention(qr, widen(kb_ref, dt, kv), widen(vb_ref, dt, kv), nh, kv, HD, pos)
            assert_close(out.numpy(), ref, what)
        else:  # batched paged layer step (its RoPE base is 1e6 in this test's call)
            n_seq = int(rng.integers(1, 6))
            positions = rng.integers(0, 1500, n_seq).astype(np.int32)
            positions[rng.random(n_seq) < 0.3] = int(rng.choice([0, 15, 16, 31]))
            k_st = [store(oracle.normal(7600 + 10 * seed + s, (int(p) + 1, kvd)), dt, kv) for s, p in
                    enumerate(positions)]
            v_st = [store(oracle.normal(7700 + 10 * seed + s, (int(p) + 1, kvd)), dt, kv) for s, p in
                    enumerate(positions)]
            n_pages = int(sum((p + PR) // PR for p in positions)) + 3
            kp, table = paged_pool(k_st, n_pages, np.random.default_rng(7800 + seed))
            vp, _ = paged_pool(v_st, n_pages, np.random.default_rng(7800 + seed))
            q = oracle.normal(7900 + seed, (n_seq, nh * HD))
            kn, vn = oracle.normal(7901 + seed, (n_seq, kvd)), oracle.normal(7902 + seed, (n_seq, kvd))
            dk, dv, out = up(kp), up(vp), ctx.empty((n_seq, nh * HD))
            dev.append(out)
            ctx.layer_attention_paged(up(q), up(kn), up(vn), dk, dv, n_pages, up(table), table.shape[1],
                                      up(positions), out, n_seq, nh, kv, HD, int(positions.max()) + 1, 1e6,
                                      kv_dtype=dt)
            got = out.numpy()
            kp_ref, vp_ref = kp.copy(), vp.copy()
            for s, p in enumerate(positions):
                qr, kr = oracle.rope(q[s], kn[s], nh, kv, HD, int(p), 1e6)
                row = table[s, p // PR] * PR + p % PR
                kp_ref[row] = store(kr, dt, kv)[0]
                vp_ref[row] = store(vn[s], dt, kv)[0]
                rows = pool_rows(table, s, int(p) + 1)
                ref = oracle.attention(qr, widen(kp_ref[rows], dt, kv), widen(vp_ref[rows], dt, kv), nh, kv, HD,
                                       int(p))
                assert_close(got[s], ref, f"{what} seq {s} pos {p}")
            np.testing.assert_array_equal(dk.numpy(), kp_ref, err_msg=what)
            np.testing.assert_array_equal(dv.numpy(), vp_ref, err_msg=what)
        assert ctx.check_device_error() == 0, what
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, 0)
        ctx.set_option(tmac_attn.TMAC_OPT_MFMA_DECODE, 1)
        ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 0)
        ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 1)
        for d in dev:
            d.free()


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("g,kv", [(4, 4), (2, 2), (8, 1), (7, 2)])
@pytest.mark.parametrize("split_len", [0, 24, 40])
def test_paged_split_lengths_align_to_pages(ctx, dt, g, kv, split_len):
    """Paged decode and the batched paged layer step on the unit grid with the
    automatic split length and with forced lengths that are not multiples of
    the 16-row page (24, 40).  A split must start on a page: the MFMA decode's
    16-row tiles and the group kernel's steps each read one page.  The
    automatic length of the 4-wave MFMA decode at 4 kv heads is a multiple of 8
    rows only (4 waves x 2 rows per step), which put split starts inside pages;
    lengths are now rounded up to a whole page on paged caches."""
    nh, kvd = g * kv, kv * HD
    lens = np.array([987, 1519, 213, 2382], np.int32)
    n_seq = lens.size
    q = oracle.normal(8500, (n_seq, nh * HD))
    k_st = [store(oracle.normal(8510 + s, (int(lens[s]), kvd)), dt, kv) for s in range(n_seq)]
    v_st = [store(oracle.normal(8520 + s, (int(lens[s]), kvd)), dt, kv) for s in range(n_seq)]
    n_pages = int(sum((l + PR - 1) // PR for l in lens)) + 4
    kp, table = paged_pool(k_st, n_pages, np.random.default_rng(85))
    vp, _ = paged_pool(v_st, n_pages, np.random.default_rng(85))
    dq, dk, dv, dtab, dl = ctx.upload(q), ctx.upload(kp), ctx.upload(vp), ctx.upload(table), ctx.upload(lens)
    out = ctx.empty((n_seq, nh * HD))
    what = f"dt={dt} g={g} kv={kv} split={split_len}"
    ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, split_len)
    ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 0)
    try:
        ctx.decode_paged(dq, dk, dv, n_pages, dtab, table.shape[1], dl, out, n_seq, nh, kv, HD, int(lens.max()),
                         kv_dtype=dt)
        offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
        ref = oracle.attention_ragged(q, np.concatenate([widen(r, dt, kv) for r in k_st]),
                                      np.concatenate([widen(r, dt, kv) for r in v_st]), offs, lens, nh, kv, HD,
                                      n_threads=8)
        assert_close(out.numpy(), ref, "paged decode " + what)
        # the layer step at the last row of each sequence
        positions = (lens - 1).astype(np.int32)
        kn, vn = oracle.normal(8530, (n_seq, kvd)), oracle.normal(8531, (n_seq, kvd))
        dkn, dvn, dpos = ctx.upload(kn), ctx.upload(vn), ctx.upload(positions)
        ctx.layer_attention_paged(dq, dkn, dvn, dk, dv, n_pages, dtab, table.shape[1], dpos, out, n_seq, nh, kv, HD,
                                  int(lens.max()), 1e6, kv_dtype=dt)
        got = out.numpy()
        kp_ref, vp_ref = kp.copy(), vp.copy()
        for s, p in enumerate(positions):
            qr, kr = oracle.rope(q[s], kn[s], nh, kv, HD, int(p), 1e6)
            row = table[s, p // PR] * PR + p % PR
            kp_ref[row] = store(kr, dt, kv)[0]
            vp_ref[row] = store(vn[s], dt, kv)[0]
            rows = pool_rows(table, s, int(p) + 1)
            ref = oracle.attention(qr, widen(kp_ref[rows], dt, kv), widen(vp_ref[rows], dt, kv), nh, kv, HD, int(p))
            assert_close(got[s], ref, f"paged layer step {what} seq {s}")
        np.testing.assert_array_equal(dk.numpy(), kp_ref, err_msg=what)
        for d in (dkn, dvn, dpos):
            d.free()
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 0)
        ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 1)
        for d in (dq, dk, dv, dtab, dl, out):
            d.free()
    assert ctx.check_device_error() == 0, what


@pytest.mark.parametrize("vs", [1, 2, 4, 8])
@pytest.mark.parametrize("g,kv", SHAPES)
def test_split_v_every_shape_and_split(ctx, g, kv, vs):
    """The split-V head kernel on every compiled shape and V split: its n_head * VS
    workgroups are dealt to the XCDs in a remapped order (contiguous runs of
    (kv head, V part, head in group) per XCD), which is a permutation of the grid
    also when the grid is not a multiple of 8 (n_head * VS = 1, 2, 4, 7, 8, 14, 16,
    28, ...).  attention_op on 1 and 300 rows, a ragged batch of two sequences
    (one of them empty) and the fused layer step (new cache rows bit for bit)."""
    nh, kvd = g * kv, kv * HD
    what = f"g={g} kv={kv} vs={vs}"
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, tmac_attn.TMAC_KERNEL_HEADV)
    ctx.set_option(tmac_attn.TMAC_OPT_HV_SPLIT, vs)
    dev = []

    def up(x):
        d = ctx.upload(x)
        dev.append(d)
        return d
    try:
        for past_len in (0, 299):
            k, v = oracle.normal(8600 + past_len, (past_len + 1, kvd)), oracle.normal(8601 + past_len, (past_len + 1, kvd))
            q = oracle.normal(8602 + past_len, nh * HD)
            out = ctx.empty(nh * HD)
            dev.append(out)
            ctx.attention_op(up(q), up(k), up(v), out, nh, kv, HD, past_len)
            assert_close(out.numpy(), oracle.attention(q, k, v, nh, kv, HD, past_len), f"{what} past_len {past_len}")
        lens = np.array([0, 77], np.int32)
        offs = np.array([0, 0], np.int64)
        k, v = oracle.normal(8610, (77, kvd)), oracle.normal(8611, (77, kvd))
        q = oracle.normal(8612, (2, nh * HD))
        out = ctx.empty((2, nh * HD))
        dev.append(out)
        ctx.decode_ragged(up(q), up(k), up(v), up(offs), up(lens), out, 2, nh, kv, HD, 77)
        got = out.numpy()
        assert np.all(got[0] == 0), what
        assert_close(got[1:], oracle.attention_ragged(q[1:], k, v, offs[1:], lens[1:], nh, kv, HD), what + " ragged")
        pos, cap = 150, 160
        kc, vc = oracle.normal(8620, (cap, kvd)), oracle.normal(8621, (cap, kvd))
        q, kn, vn = oracle.normal(8622, nh * HD), oracle.normal(8623, kvd), oracle.normal(8624, kvd)
        dkc, dvc, out = up(kc), up(vc), ctx.empty(nh * HD)
        dev.append(out)
        ctx.layer_attention(up(q), up(kn), up(vn), dkc, dvc, out, nh, kv, HD, pos, cap, 1e6)
        kc_ref, vc_ref = kc.copy(), vc.copy()
        ref, _, _ = oracle.layer_step(q, kn, vn, kc_ref, vc_ref, nh, kv, HD, pos, 1e6)  # updates the copies
        assert_close(out.numpy(), ref, what + " layer step")
        np.testing.assert_array_equal(dkc.numpy(), kc_ref, err_msg=what)
        np.testing.assert_array_equal(dvc.numpy(), vc_ref, err_msg=what)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, tmac_attn.TMAC_KERNEL_AUTO)
        ctx.set_option(tmac_attn.TMAC_OPT_HV_SPLIT, 8)
        for d in dev:
            d.free()
    assert ctx.check_device_error() == 0, what
