"""GPU parity of the bf16-MFMA chunked causal prefill.

Oracle: the reference's decode applied per query row (tmac_gguf.cpp:1093-1128
with past_len = prefix + i), fed the bf16-rounded q/k/v the kernel computes
with (config 5 takes bf16 MFMA operands, so the parity inputs are the
bf16-rounded ones).  Tolerance: the fp32 bound |gpu - ref| <= 2e-5 + 1e-4 |ref|.
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close

pytestmark = pytest.mark.gpu
HD = 64


def bf16_round(x):
    """Round-to-nearest-even to bfloat16, returned as float32 (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


def make(seed, n_seq, n_q, prefix, cap, n_head, n_kv):
    q = oracle.normal(seed, (n_seq, n_q, n_head * HD))
    k = oracle.normal(seed + 1, (n_seq, cap, n_kv * HD))
    v = oracle.normal(seed + 2, (n_seq, cap, n_kv * HD))
    return q, k, v


def run(ctx, q, k, v, n_seq, n_q, prefix, cap, n_head, n_kv):
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    out = ctx.empty((n_seq, n_q, n_head * HD))
    ctx.prefill(dq, dk, dv, out, n_seq, n_q, prefix, cap, n_head, n_kv, HD)
    return out.numpy()


@pytest.mark.parametrize("n_seq,n_q,prefix,n_head,n_kv", [
    (1, 1, 0, 14, 2), (1, 5, 0, 14, 2), (2, 37, 100, 14, 2), (1, 64, 63, 14, 2),
    (3, 16, 17, 14, 2), (1, 33, 200, 16, 4), (2, 20, 50, 8, 1), (1, 48, 31, 2, 2), (1, 17, 5, 1, 1)])
def test_prefill_bf16_exact_inputs(ctx, n_seq, n_q, prefix, n_head, n_kv):
    cap = prefix + n_q + 3
    q, k, v = (bf16_round(a) for a in make(500 + n_q, n_seq, n_q, prefix, cap, n_head, n_kv))
    got = run(ctx, q, k, v, n_seq, n_q, prefix, cap, n_head, n_kv)
    ref = oracle.prefill(q, k, v, n_seq, n_q, prefix, cap, n_head, n_kv, HD, n_threads=8)
    assert_close(got, ref, f"prefill {n_seq}x{n_q} prefix {prefix} heads {n_head}/{n_kv}")


def test_prefill_rounds_fp32_inputs_to_nearest_even(ctx):
    """Raw fp32 inputs: the kernel's own bf16 conversion must equal round-to-nearest-even."""
    n_seq, n_q, prefix, cap = 2, 40, 90, 140
    q, k, v = make(600, n_seq, n_q, prefix, cap, 14, 2)
    got = run(ctx, q, k, v, n_seq, n_q, prefix, cap, 14, 2)
    ref = oracle.prefill(bf16_round(q), bf16_round(k), bf16_round(v), n_seq, n_q, prefix, cap, 14, 2, HD, n_threads=8)
    assert_close(got, ref, "prefill raw fp32 inputs vs oracle on bf16-rounded inputs")
    # and the bf16 input rounding is visible against the unrounded oracle (stated, looser bound)
    raw = oracle.prefill(q, k, v, n_seq, n_q, prefix, cap, 14, 2, HD, n_threads=8)
    err = np.abs(got - raw)
    assert err.max() < 2e-2 and err.max() > 1e-5


def test_prefill_config5_sampled_rows(ctx):
    """Config 5 shape: 4 sequences x 512-query chunk after a 1536-row prefix (context 2048);
    every 8th query row of every sequence is checked against the oracle."""
    n_seq, n_q, prefix, cap = 4, 512, 1536, 2048
    rng = np.random.default_rng(5)
    q = bf16_round(rng.standard_normal((n_seq, n_q, 14 * HD), dtype=np.float32))
    k = bf16_round(rng.standard_normal((n_seq, cap, 2 * HD), dtype=np.float32))
    v = bf16_round(rng.standard_normal((n_seq, cap, 2 * HD), dtype=np.float32))
    got = run(ctx, q, k, v, n_seq, n_q, prefix, cap, 14, 2)
    rows = np.arange(0, n_q, 8)
    offs = np.concatenate([s * cap + np.zeros(rows.size, np.int64) for s in range(n_seq)])
    lens = np.concatenate([prefix + rows + 1 for _ in range(n_seq)]).astype(np.int32)
    qs = np.concatenate([q[s, rows] for s in range(n_seq)])
    ref = oracle.attention_ragged(qs, k.reshape(-1, 2 * HD), v.reshape(-1, 2 * HD), offs, lens, 14, 2, HD,
                                  n_threads=16)
    assert_close(np.concatenate([got[s, rows] for s in range(n_seq)]), ref, "config 5 sampled rows")


@pytest.mark.parametrize("dt", ["bf16", "f16", "q8"])
@pytest.mark.parametrize("n_seq,n_q,prefix,n_head,n_kv", [(2, 37, 100, 14, 2), (1, 33, 200, 16, 4),
                                                          (2, 20, 50, 8, 1), (1, 5, 0, 14, 2)])
def test_prefill_narrow_caches(ctx, dt, n_seq, n_q, prefix, n_head, n_kv):
    """tmac_attention_prefill_kv over a bf16 / fp16 / Q8_0 cache: the rows are
    widened exactly to fp32, then rounded to bf16 like fp32 rows, so the
    reference is the oracle on those widened, rounded rows."""
    import tmac_attn
    cap = prefix + n_q + 3
    q, k, v = make(800 + n_q, n_seq, n_q, prefix, cap, n_head, n_kv)
    q = bf16_round(q)
    kvd = n_kv * HD
    if dt == "bf16":
        code = tmac_attn.TMAC_KV_BF16
        store = lambda x: (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)
        widen = lambda b: (b.astype(np.uint32) << 16).view(np.float32)
    elif dt == "f16":
        code = tmac_attn.TMAC_KV_F16
        store = lambda x: x.astype(np.float16).view(np.uint16)
        widen = lambda b: b.view(np.float16).astype(np.float32)
    else:
        code = tmac_attn.TMAC_KV_Q8_0
        store = lambda x: oracle.q8_kv_rows(x.reshape(-1, HD)).reshape(n_seq, cap, n_kv * oracle.Q8_HEAD_BYTES)
        widen = lambda b: oracle.q8_kv_widen(b).reshape(n_seq, cap, kvd)
    kb, vb = store(k), store(v)
    kw, vw = bf16_round(widen(kb).reshape(n_seq, cap, kvd)), bf16_round(widen(vb).reshape(n_seq, cap, kvd))
    dq, dk, dv = ctx.upload(q), ctx.upload(kb), ctx.upload(vb)
    out = ctx.empty((n_seq, n_q, n_head * HD))
    ctx.prefill(dq, dk, dv, out, n_seq, n_q, prefix, cap, n_head, n_kv, HD, kv_dtype=code)
    ref = oracle.prefill(q, kw, vw, n_seq, n_q, prefix, cap, n_head, n_kv, HD, n_threads=8)
    assert_close(out.numpy(), ref, f"prefill {dt} {n_seq}x{n_q} prefix {prefix} heads {n_head}/{n_kv}")
    assert ctx.prefill(dq, dk, dv, out, n_seq, n_q, prefix, cap, n_head, n_kv, HD, kv_dtype=9,
                       check=False) == tmac_attn.TMAC_ERR_INVALID_ARG


@pytest.mark.parametrize("dt", ["f32", "bf16", "q8"])
def test_prefill_paged(ctx, dt):
    """tmac_attention_prefill_paged: the rows of 3 sequences scattered over a
    pool of 16-row pages in random order (sequence 1 sharing sequence 0's
    first 4 pages) give what the contiguous prefill gives on the same rows."""
    import tmac_attn
    n_seq, n_q, prefix, n_head, n_kv, pr = 3, 40, 90, 14, 2, tmac_attn.PAGE_ROWS
    rows = prefix + n_q
    kvd = n_kv * HD
    q, k, v = make(900, n_seq, n_q, prefix, rows, n_head, n_kv)
    k[1, :4 * pr], v[1, :4 * pr] = k[0, :4 * pr], v[0, :4 * pr]  # the shared prefix pages hold equal rows
    q = bf16_round(q)
    if dt == "f32":
        code, store, widen = tmac_attn.TMAC_KV_F32, (lambda x: x), (lambda b: b)
    elif dt == "bf16":
        code = tmac_attn.TMAC_KV_BF16
        store = lambda x: (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)
        widen = lambda b: (b.astype(np.uint32) << 16).view(np.float32)
    else:
        code = tmac_attn.TMAC_KV_Q8_0
        store = lambda x: oracle.q8_kv_rows(x.reshape(-1, HD)).reshape(*x.shape[:-1], n_kv * oracle.Q8_HEAD_BYTES)
        widen = lambda b: oracle.q8_kv_widen(b).reshape(*b.shape[:-1], kvd)
    kb, vb = store(k), store(v)
    max_pages = (rows + pr - 1) // pr
    n_pages = n_seq * max_pages + 5
    rng = np.random.default_rng(9)
    perm = rng.permutation(n_pages)
    table = np.zeros((n_seq, max_pages), np.int32)
    kp = np.zeros((n_pages * pr,) + kb.shape[2:], kb.dtype)
    vp = np.zeros_like(kp)
    nxt = 0
    for s in range(n_seq):
        for j in range(max_pages):
            if s == 1 and j < 4:
                table[s, j] = table[0, j]
                continue
            table[s, j] = perm[nxt]
            nxt += 1
            seg = slice(j * pr, min(rows, (j + 1) * pr))
            kp[table[s, j] * pr:table[s, j] * pr + seg.stop - seg.start] = kb[s, seg]
            vp[table[s, j] * pr:table[s, j] * pr + seg.stop - seg.start] = vb[s, seg]
    dq, dk, dv, dtab = ctx.upload(q), ctx.upload(kp), ctx.upload(vp), ctx.upload(table)
    out = ctx.empty((n_seq, n_q, n_head * HD))
    ctx.prefill_paged(dq, dk, dv, n_pages, dtab, max_pages, out, n_seq, n_q, prefix, n_head, n_kv, HD, kv_dtype=code)
    kw = bf16_round(np.asarray(widen(kb), np.float32).reshape(n_seq, rows, kvd))
    vw = bf16_round(np.asarray(widen(vb), np.float32).reshape(n_seq, rows, kvd))
    ref = oracle.prefill(q, kw, vw, n_seq, n_q, prefix, rows, n_head, n_kv, HD, n_threads=8)
    assert_close(out.numpy(), ref, f"paged prefill {dt}")
    assert ctx.check_device_error() == 0
    # an entry outside the pool is clamped (no out-of-bounds read) and reported (bit 2)
    bad = table.copy()
    bad[2, 3] = n_pages + 7
    ctx.prefill_paged(dq, dk, dv, n_pages, ctx.upload(bad), max_pages, out, n_seq, n_q, prefix, n_head, n_kv, HD,
                      kv_dtype=code)
    assert ctx.check_device_error() == tmac_attn.TMAC_ERR_DEVICE_FAULT
    assert ctx.prefill_paged(dq, dk, dv, n_pages, dtab, 2, out, n_seq, n_q, prefix, n_head, n_kv, HD,
                             kv_dtype=code, check=False) == tmac_attn.TMAC_ERR_INVALID_ARG  # rows > 16 * max_pages


@pytest.mark.parametrize("dt", ["f32", "q8"])
def test_chunked_prompt_rope_rows_write_prefill(ctx, dt):
    """A 300-token prompt fed in 64-token chunks the way a caller would:
    tmac_rope_rows rotates the chunk's q and k rows, the rotated k and v rows
    go into the cache (a device copy for fp32, tmac_kv_convert for Q8_0), and
    the chunk's prefill attends rows 0..its position.  The cache rows equal
    the oracle's RoPE (tmac_gguf.cpp:990-1016) and Q8_0 rule bit for bit; the
    outputs equal the oracle's attention on the bf16-rounded rotated rows."""
    import ctypes
    import tmac_attn
    nh, nkv, n_tok, chunk = 14, 2, 300, 64
    kvd = nkv * HD
    cap = 320
    q_all = oracle.normal(950, (n_tok, nh * HD))
    k_all = oracle.normal(951, (n_tok, kvd))
    v_all = oracle.normal(952, (n_tok, kvd))
    q8 = dt == "q8"
    rb = nkv * oracle.Q8_HEAD_BYTES if q8 else kvd
    dk = ctx.upload(np.zeros((cap, rb), np.uint8 if q8 else np.float32))
    dv = ctx.upload(np.zeros((cap, rb), np.uint8 if q8 else np.float32))
    ref_k = np.zeros((cap, kvd), np.float32)  # rotated rows as the cache holds them (widened)
    ref_v = np.zeros((cap, kvd), np.float32)
    ref_k_bytes = np.zeros((cap, rb), np.uint8 if q8 else np.float32)
    for c0 in range(0, n_tok, chunk):
        n = min(chunk, n_tok - c0)
        dq, dkc, dvc = ctx.upload(q_all[c0:c0 + n]), ctx.upload(k_all[c0:c0 + n]), ctx.upload(v_all[c0:c0 + n])
        ctx.rope_rows(dq, n, nh * HD, nh, HD, c0, 1e6)
        ctx.rope_rows(dkc, n, kvd, nkv, HD, c0, 1e6)
        if q8:
            ctx.kv_convert(tmac_attn.TMAC_KV_Q8_0, dkc, dk.at(c0 * rb), n * kvd)
            ctx.kv_convert(tmac_attn.TMAC_KV_Q8_0, dvc, dv.at(c0 * rb), n * kvd)
        else:
            for src, dst in ((dkc, dk), (dvc, dv)):
                rc = ctx.lib.tmac_memcpy_d2d(ctx.handle, None, ctypes.c_void_p(dst.at(c0 * kvd)),
                                             ctypes.c_void_p(src.ptr), n * kvd * 4)
                assert rc == 0
        out = ctx.empty((1, n, nh * HD))
        ctx.prefill(dq, dk, dv, out, 1, n, c0, cap, nh, nkv, HD, kv_dtype=tmac_attn.TMAC_KV_Q8_0 if q8 else 0)
        q_rot = np.empty((n, nh * HD), np.float32)
        for i in range(n):
            qr, kr = oracle.rope(q_all[c0 + i], k_all[c0 + i], nh, nkv, HD, c0 + i, 1e6)
            q_rot[i] = qr
            if q8:
                ref_k_bytes[c0 + i] = oracle.q8_kv_rows(kr.reshape(-1, HD)).reshape(-1)
                ref_k[c0 + i] = oracle.q8_kv_widen(ref_k_bytes[c0 + i]).reshape(-1)
                ref_v[c0 + i] = oracle.q8_kv_widen(oracle.q8_kv_rows(v_all[c0 + i].reshape(-1, HD))).reshape(-1)
            else:
                ref_k_bytes[c0 + i] = kr
                ref_k[c0 + i], ref_v[c0 + i] = kr, v_all[c0 + i]
        np.testing.assert_array_equal(dq.numpy(), q_rot)  # the chunk RoPE, bit for bit
        ref = oracle.prefill(bf16_round(q_rot)[None], bf16_round(ref_k)[None], bf16_round(ref_v)[None], 1, n, c0,
                             cap, nh, nkv, HD, n_threads=8)
        assert_close(out.numpy(), ref, f"chunk at {c0} ({dt})")
    np.testing.assert_array_equal(dk.numpy()[:n_tok], ref_k_bytes[:n_tok])
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("dt", ["f32", "bf16", "q8"])
def test_prefill_tiles_chunks_match_full_call(ctx, dt):
    """Chunked prefill over the persistent tile copy: each chunk packs only its
    own rows (tmac_prefill_pack_rows, chunk starts not on 64-row tiles) and
    attends through tmac_attention_prefill_tiles.  Every chunk's outputs equal
    tmac_attention_prefill's on the same cache bit for bit, and the oracle's on
    the bf16-rounded inputs within the fp32 tolerance."""
    import tmac_attn
    n_seq, nh, nkv, cap = 2, 14, 2, 700
    q, k, v = (bf16_round(a) for a in make(970, n_seq, cap, 0, cap, nh, nkv))
    code = {"f32": tmac_attn.TMAC_KV_F32, "bf16": tmac_attn.TMAC_KV_BF16, "q8": tmac_attn.TMAC_KV_Q8_0}[dt]
    if dt == "f32":
        kb, vb, kw, vw = k, v, k, v
    elif dt == "bf16":  # bf16-exact values: the cache holds them exactly
        kb, vb = ((x.view(np.uint32) >> 16).astype(np.uint16) for x in (k, v))
        kw, vw = k, v
    else:
        kb, vb = (oracle.q8_kv_rows(x.reshape(-1, HD)).reshape(n_seq, cap, nkv * oracle.Q8_HEAD_BYTES) for x in (k, v))
        kw, vw = (bf16_round(oracle.q8_kv_widen(b).reshape(n_seq, cap, nkv * HD)) for b in (kb, vb))
    dk, dv = ctx.upload(kb), ctx.upload(vb)
    tiles = ctx.empty(ctx.prefill_tiles_bytes(n_seq, nkv, cap), np.uint8)
    for c0, c1 in ((0, 200), (200, 450), (450, 700)):
        n = c1 - c0
        dq = ctx.upload(np.ascontiguousarray(q[:, c0:c1]))
        ctx.prefill_pack_rows(dk, dv, cap, tiles, cap, n_seq, nkv, HD, c0, c1, kv_dtype=code)
        out_t, out_f = ctx.empty((n_seq, n, nh * HD)), ctx.empty((n_seq, n, nh * HD))
        ctx.prefill_tiles(dq, tiles, cap, out_t, n_seq, n, c0, nh, nkv, HD)
        ctx.prefill(dq, dk, dv, out_f, n_seq, n, c0, cap, nh, nkv, HD, kv_dtype=code)
        got = out_t.numpy()
        np.testing.assert_array_equal(got.view(np.uint32), out_f.numpy().view(np.uint32), err_msg=f"chunk {c0} {dt}")
        ref = oracle.prefill(np.ascontiguousarray(q[:, c0:c1]), kw, vw, n_seq, n, c0, cap, nh, nkv, HD, n_threads=8)
        assert_close(got, ref, f"chunk {c0} ({dt}) vs oracle")
    assert ctx.check_device_error() == 0


def test_prefill_tiles_repack_middle_range_and_unwritten_rows(ctx):
    """tmac_prefill_pack_rows writes only the rows it is given.  The tile buffer
    starts as all-ones bytes (every bf16 a NaN): (1) after packing only rows
    0..129, a chunk ending at row 130 reads tile 2, whose rows 130..191 were never
    written, and still equals tmac_attention_prefill bit for bit; (2) with every
    row packed back to front, cache rows 100..109 are then changed and only they
    are repacked, and chunks ending past row 110 (which reads tile 1's rows
    110..127, packed earlier) equal tmac_attention_prefill on the changed cache bit
    for bit and the oracle within the fp32 tolerance."""
    n_seq, nh, nkv, cap = 2, 14, 2, 300
    q, k, v = (bf16_round(a) for a in make(990, n_seq, cap, 0, cap, nh, nkv))
    dk, dv = ctx.upload(k), ctx.upload(v)
    tiles = ctx.empty(ctx.prefill_tiles_bytes(n_seq, nkv, cap), np.uint8)
    tiles.fill_bytes(0xFF)

    def check(c0, c1, kk, vv, what):
        n = c1 - c0
        dq = ctx.upload(np.ascontiguousarray(q[:, c0:c1]))
        out_t, out_f = ctx.empty((n_seq, n, nh * HD)), ctx.empty((n_seq, n, nh * HD))
        ctx.prefill_tiles(dq, tiles, cap, out_t, n_seq, n, c0, nh, nkv, HD)
        ctx.prefill(dq, dk, dv, out_f, n_seq, n, c0, cap, nh, nkv, HD)
        got = out_t.numpy()
        assert np.all(np.isfinite(got)), what
        np.testing.assert_array_equal(got.view(np.uint32), out_f.numpy().view(np.uint32), err_msg=what)
        ref = oracle.prefill(np.ascontiguousarray(q[:, c0:c1]), kk, vv, n_seq, n, c0, cap, nh, nkv, HD, n_threads=8)
        assert_close(got, ref, what)
        for d in (dq, out_t, out_f):
            d.free()

    ctx.prefill_pack_rows(dk, dv, cap, tiles, cap, n_seq, nkv, HD, 0, 130)
    check(100, 130, k, v, "rows 130..191 of tile 2 never packed")
    for r0, r1 in ((250, 300), (130, 250), (0, 130)):  # back to front
        ctx.prefill_pack_rows(dk, dv, cap, tiles, cap, n_seq, nkv, HD, r0, r1)
    k2, v2 = k.copy(), v.copy()
    k2[:, 100:110] = bf16_round(oracle.normal(995, (n_seq, 10, nkv * HD)) * 3)
    v2[:, 100:110] = bf16_round(oracle.normal(996, (n_seq, 10, nkv * HD)))
    dk.copy_from(k2)
    dv.copy_from(v2)
    ctx.prefill_pack_rows(dk, dv, cap, tiles, cap, n_seq, nkv, HD, 100, 110)
    for c0, c1 in ((0, 300), (105, 140), (120, 128)):
        check(c0, c1, k2, v2, f"chunk {c0}..{c1} after rows 100..109 were repacked")
    for d in (dk, dv, tiles):
        d.free()
    assert ctx.check_device_error() == 0


def test_prefill_tiles_rejects_bad_arguments(ctx):
    import tmac_attn
    d = ctx.empty(4096)
    cap = 100
    tiles = ctx.empty(ctx.prefill_tiles_bytes(2, 2, cap), np.uint8)
    bad = tmac_attn.TMAC_ERR_INVALID_ARG
    assert ctx.prefill_pack_rows(d, d, cap, tiles, cap, 2, 2, HD, 0, cap + 1, check=False) == bad  # past capacity
    assert ctx.prefill_pack_rows(d, d, cap, tiles, cap, 2, 2, HD, 10, 5, check=False) == bad  # end before begin
    assert ctx.prefill_pack_rows(d, d, cap - 1, tiles, cap, 2, 2, HD, 0, 10, check=False) == bad  # stride < capacity
    assert ctx.prefill_pack_rows(d, d, cap, tiles, cap, 2, 2, 32, 0, 10, check=False) == tmac_attn.TMAC_ERR_UNSUPPORTED
    assert ctx.prefill_tiles(d, tiles, cap, d, 2, 60, 50, 14, 2, HD, check=False) == bad  # rows past capacity
    assert ctx.prefill_tiles(d, tiles, cap, d, 2, 10, 0, 14, 3, HD, check=False) == bad
    assert ctx.prefill_tiles(d, None, cap, d, 2, 10, 0, 14, 2, HD, check=False) == tmac_attn.TMAC_ERR_NULL_POINTER
    assert ctx.prefill_tiles_bytes(2, 2, cap) == 2 * 2 * 4 * 64 * 64 * 2 * 2  # 100 rows -> 4 tiles (one stage)
    assert ctx.check_device_error() == 0


def test_prefill_rejects_bad_arguments(ctx):
    import tmac_attn
    d = ctx.empty(16 * 14 * HD)
    assert ctx.prefill(d, d, d, d, 2, 16, 10, 20, 14, 2, HD, check=False) == tmac_attn.TMAC_ERR_INVALID_ARG
    assert ctx.prefill(d, d, d, d, 1, 16, 0, 16, 14, 2, 32, check=False) == tmac_attn.TMAC_ERR_UNSUPPORTED
    assert ctx.prefill(d, d, d, d, 1, 16, 0, 16, 14, 3, HD, check=False) == tmac_attn.TMAC_ERR_INVALID_ARG


def test_prefill_graph_replay_matches_eager(ctx):
    """Both prefill launches (tile pack + attention) captured into a graph: every
    replay, with eager calls and new queries in between, equals the eager call
    on the same inputs bit for bit, and the first also the oracle."""
    n_seq, n_q, prefix, cap = 2, 40, 70, 120
    q, k, v = (bf16_round(a) for a in make(700, n_seq, n_q, prefix, cap, 14, 2))
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    out_e = ctx.empty((n_seq, n_q, 14 * HD))
    out_g = ctx.empty((n_seq, n_q, 14 * HD))
    s = ctx.stream()
    ctx.prefill(dq, dk, dv, out_e, n_seq, n_q, prefix, cap, 14, 2, HD, stream=s)  # sizes the workspace
    ctx.synchronize(s)
    ctx.step_begin(s)
    ctx.prefill(dq, dk, dv, out_g, n_seq, n_q, prefix, cap, 14, 2, HD, stream=s)
    g = ctx.step_end(s)
    try:
        for rep in range(3):
            qn = bf16_round(oracle.normal(710 + rep, (n_seq, n_q, 14 * HD)))
            dq.copy_from(qn)
            ctx.prefill(dq, dk, dv, out_e, n_seq, n_q, prefix, cap, 14, 2, HD, stream=s)
            ctx.synchronize(s)
            ctx.graph_launch(g, s)
            ctx.synchronize(s)
            got = out_g.numpy()
            np.testing.assert_array_equal(got, out_e.numpy(), err_msg=f"replay {rep}")
            if rep == 0:
                ref = oracle.prefill(qn, k, v, n_seq, n_q, prefix, cap, 14, 2, HD, n_threads=8)
                assert_close(got, ref, "graph replay vs oracle")
    finally:
        ctx.graph_destroy(g)
        ctx.destroy_stream(s)


@pytest.mark.parametrize("seed", range(10))
def test_prefill_random_cases(ctx, seed):
    """Seeded random chunked prefills: 1-3 sequences, 1-200 queries after a
    0-700-row prefix, spare capacity, and a GQA shape drawn from the compiled
    ones, on bf16-exact inputs (the kernel's operands are then the inputs)."""
    rng = np.random.default_rng(3000 + seed)
    n_head, n_kv = [(14, 2), (16, 4), (8, 1), (2, 2), (1, 1), (4, 2)][seed % 6]
    n_seq = int(rng.integers(1, 4))
    n_q = int(rng.integers(1, 201))
    prefix = int(rng.choice([0, int(rng.integers(1, 64)), int(rng.integers(64, 701))]))
    cap = prefix + n_q + int(rng.integers(0, 30))
    q, k, v = (bf16_round(a) for a in make(3100 + 10 * seed, n_seq, n_q, prefix, cap, n_head, n_kv))
    got = run(ctx, q, k, v, n_seq, n_q, prefix, cap, n_head, n_kv)
    ref = oracle.prefill(q, k, v, n_seq, n_q, prefix, cap, n_head, n_kv, HD, n_threads=8)
    assert_close(got, ref, f"seed {seed}: {n_seq}x{n_q} prefix {prefix} cap {cap} heads {n_head}/{n_kv}")
