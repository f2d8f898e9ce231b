"""GPU parity of the Q8_0 KV cache (TMAC_KV_Q8_0, tmac_kv_convert) and of the
paged caches (tmac_attention_decode_paged, tmac_layer_attention_paged) for
every cache element type.

Contract: a cache row is read and widened exactly to fp32, so every output
must equal the oracle's attention (tmac_gguf.cpp:1093-1128) on the widened
rows within the fp32 tolerance |gpu - ref| <= 2e-5 + 1e-4 |ref|.  Bytes the
kernels write are checked bit for bit: a Q8_0 row against the oracle's
restatement of the reference's quantize_q8_0_block
(scripts/extract_tmac.py:159-173), a bf16/fp16 row against numpy's
nearest-even rounding, an fp32 row against the oracle's RoPE
(tmac_gguf.cpp:990-1016).  A paged cache must give exactly what the
contiguous cache holding the same rows gives: the oracle sees the rows
gathered through the block table.
"""
import numpy as np
import pytest

import oracle
import tmac_attn
from conftest import assert_close

pytestmark = pytest.mark.gpu
NH, NKV, HD = 14, 2, 64
KVD = NKV * HD
PR = tmac_attn.PAGE_ROWS
Q8 = tmac_attn.TMAC_KV_Q8_0
ALL_DT = [tmac_attn.TMAC_KV_F32, tmac_attn.TMAC_KV_BF16, tmac_attn.TMAC_KV_F16, Q8]


def store(x: np.ndarray, dt: int) -> np.ndarray:
    """fp32 rows [n, KVD] -> the cache's stored rows (fp32, uint16 or uint8 [n, NKV * 68])."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, KVD)
    if dt == tmac_attn.TMAC_KV_F32:
        return x.copy()
    if dt == tmac_attn.TMAC_KV_F16:
        return x.astype(np.float16).view(np.uint16)
    if dt == tmac_attn.TMAC_KV_BF16:
        u = x.view(np.uint32).astype(np.uint64)
        return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)
    return oracle.q8_kv_rows(x).reshape(-1, NKV * oracle.Q8_HEAD_BYTES)


def widen(rows: np.ndarray, dt: int) -> np.ndarray:
    """Stored rows -> fp32 [n, KVD], exactly."""
    if dt == tmac_attn.TMAC_KV_F32:
        return np.asarray(rows, np.float32).reshape(-1, KVD)
    if dt == tmac_attn.TMAC_KV_F16:
        return np.ascontiguousarray(rows, np.uint16).view(np.float16).astype(np.float32).reshape(-1, KVD)
    if dt == tmac_attn.TMAC_KV_BF16:
        return (np.ascontiguousarray(rows, np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(-1, KVD)
    return oracle.q8_kv_widen(rows).reshape(-1, KVD)


def data(seed, shape, scale_spread=0.0):
    x = oracle.normal(seed, shape)
    if scale_spread:  # rows of very different magnitudes (exercises the Q8_0 block scales)
        rng = np.random.default_rng(seed)
        x = x * np.exp2(rng.uniform(-scale_spread, scale_spread, x.shape[:-1] + (1,))).astype(np.float32)
    return x.astype(np.float32)


# ---- Q8_0 cache ---------------------------------------------------------------------------------

def test_kv_convert_q8_bit_exact(ctx):
    x = data(60, (3000, 64), scale_spread=12)
    x[0] = 0.0                           # all-zero block pair: d = 1, q = 0
    x[1, :32] = 1e-12                    # max |x| < 1e-10: d = 1
    x[2, 5] = 127.0                      # d = 1 exactly: q = x rounded half to even
    x[2, 6:10] = [0.5, 1.5, 2.5, -0.5]
    x[3] *= 1e4                          # scale above fp16's range for some blocks: d -> inf bits
    dx, dy = ctx.upload(x), ctx.empty((x.shape[0], oracle.Q8_HEAD_BYTES), np.uint8)
    ctx.kv_convert(Q8, dx, dy, x.size)
    np.testing.assert_array_equal(dy.numpy(), oracle.q8_kv_rows(x))


def test_kv_convert_q8_rejects(ctx):
    d = ctx.empty(256)
    assert ctx.kv_convert(Q8, d, d, 100, check=False) == tmac_attn.TMAC_ERR_INVALID_ARG  # not a multiple of 64
    assert ctx.kv_convert(Q8, d.at(1), d, 64, check=False) == tmac_attn.TMAC_ERR_MISALIGNED


@pytest.mark.parametrize("mfma", [0, 1])
@pytest.mark.parametrize("n_seq,n_pos,kernel", [(3, 300, tmac_attn.TMAC_KERNEL_AUTO), (2, 2000, 0), (8, 4096, 0),
                                                (1, 700, tmac_attn.TMAC_KERNEL_HEAD),
                                                (2, 77, tmac_attn.TMAC_KERNEL_GROUP), (3, 17, 0), (2, 1, 0)])
def test_decode_batched_q8(ctx, mfma, n_seq, n_pos, kernel):
    q = data(800 + n_pos, (n_seq, NH * HD))
    kb = store(data(801 + n_pos, (n_seq * n_pos, KVD), 2), Q8)
    vb = store(data(802 + n_pos, (n_seq * n_pos, KVD), 2), Q8)
    dq, dk, dv, dout = ctx.upload(q), ctx.upload(kb), ctx.upload(vb), ctx.empty((n_seq, NH * HD))
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, kernel)
    ctx.set_option(tmac_attn.TMAC_OPT_MFMA_DECODE, mfma)
    try:
        ctx.decode_batched(dq, dk, dv, dout, n_seq, NH, NKV, HD, n_pos, n_pos, kv_dtype=Q8)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, 0)
        ctx.set_option(tmac_attn.TMAC_OPT_MFMA_DECODE, 1)
    offs = np.arange(n_seq, dtype=np.int64) * n_pos
    lens = np.full(n_seq, n_pos, np.int32)
    ref = oracle.attention_ragged(q, widen(kb, Q8), widen(vb, Q8), offs, lens, NH, NKV, HD, n_threads=8)
    assert_close(dout.numpy(), ref, f"batched q8 {n_seq}x{n_pos} mfma={mfma}")


@pytest.mark.parametrize("dt", [tmac_attn.TMAC_KV_BF16, tmac_attn.TMAC_KV_F16, Q8])
@pytest.mark.parametrize("n_pos", [336, 512, 695, 2085])
def test_decode_mfma_long_splits(ctx, dt, n_pos):
    """One split per sequence (a split length covering it), so every wave of
    the MFMA decode runs its tile loop over many tiles: 336 rows give the
    waves 2-3 full tiles, 512 rows 4 (bf16 / fp16: 8), 695 rows 5-6 and a
    7-row tail, 2085 rows 16-17 and a 5-row tail; the loop's steady state and
    each of its drain lengths are taken.  Automatic splits of these short
    batches give a wave at most one tile."""
    n_seq = 2
    q = data(830 + n_pos, (n_seq, NH * HD))
    kb = store(data(831 + n_pos, (n_seq * n_pos, KVD), 2), dt)
    vb = store(data(832 + n_pos, (n_seq * n_pos, KVD), 2), dt)
    dq, dk, dv, dout = ctx.upload(q), ctx.upload(kb), ctx.upload(vb), ctx.empty((n_seq, NH * HD))
    ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 4096)
    try:
        ctx.decode_batched(dq, dk, dv, dout, n_seq, NH, NKV, HD, n_pos, n_pos, kv_dtype=dt)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 0)
    offs = np.arange(n_seq, dtype=np.int64) * n_pos
    lens = np.full(n_seq, n_pos, np.int32)
    ref = oracle.attention_ragged(q, widen(kb, dt), widen(vb, dt), offs, lens, NH, NKV, HD, n_threads=8)
    assert_close(dout.numpy(), ref, f"dt={dt} {n_seq}x{n_pos} one split")
    assert ctx.check_device_error() == 0


def test_decode_ragged_q8(ctx):
    lens = np.array([1, 0, 513, 4000, 37, 2048, 3], np.int32)
    n_seq = lens.size
    offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64) + 5
    rows = int(offs[-1] + lens[-1])
    q = data(900, (n_seq, NH * HD))
    kb, vb = store(data(901, (rows, KVD), 2), Q8), store(data(902, (rows, KVD), 2), Q8)
    dq, dk, dv = ctx.upload(q), ctx.upload(kb), ctx.upload(vb)
    doffs, dlens, dout = ctx.upload(offs), ctx.upload(lens), ctx.empty((n_seq, NH * HD))
    for hint in (0, int(lens.sum())):
        ctx.decode_ragged(dq, dk, dv, doffs, dlens, dout, n_seq, NH, NKV, HD, int(lens.max()), hint, kv_dtype=Q8)
        nz = lens > 0
        ref = oracle.attention_ragged(q[nz], widen(kb, Q8), widen(vb, Q8), offs[nz], lens[nz], NH, NKV, HD,
                                      n_threads=8)
        got = dout.numpy()
        assert np.all(got[~nz] == 0)
        assert_close(got[nz], ref, f"ragged q8 hint={hint}")
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("seed", range(12))
def test_decode_ragged_random_cases(ctx, seed):
    """Seeded random ragged batches on every cache type: 1-6 sequences of
    0-3000 rows at gapped offsets, a random split length (automatic, 16 to
    4096 rows) and schedule (unit grid, automatic, stream-K), with and without
    the total_rows hint."""
    rng = np.random.default_rng(1000 + seed)
    dt = ALL_DT[seed % len(ALL_DT)]
    n_seq = int(rng.integers(1, 7))
    lens = rng.integers(0, 3001, n_seq).astype(np.int32)
    lens[rng.random(n_seq) < 0.15] = 0
    gaps = rng.integers(0, 40, n_seq)
    offs = (np.concatenate([[0], np.cumsum(lens[:-1])]) + np.cumsum(gaps)).astype(np.int64)
    rows = int(offs[-1] + lens[-1]) + 1
    split_len = int(rng.choice([0, 16, 48, 256, 4096]))
    stream_k = int(rng.choice([0, 1, 2]))
    hint = int(lens.sum()) if rng.random() < 0.5 else 0
    q = data(1100 + seed, (n_seq, NH * HD)) * np.float32(rng.choice([0.25, 1.0, 4.0]))
    kb = store(data(1200 + seed, (rows, KVD), 2), dt)
    vb = store(data(1300 + seed, (rows, KVD), 2), dt)
    dq, dk, dv = ctx.upload(q), ctx.upload(kb), ctx.upload(vb)
    doffs, dlens, dout = ctx.upload(offs), ctx.upload(lens), ctx.empty((n_seq, NH * HD))
    ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, split_len)
    ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, stream_k)
    try:
        ctx.decode_ragged(dq, dk, dv, doffs, dlens, dout, n_seq, NH, NKV, HD, max(int(lens.max()), 1), hint,
                          kv_dtype=dt)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 0)
        ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 1)
    what = f"seed {seed}: dt={dt} lens={lens.tolist()} split={split_len} stream_k={stream_k} hint={hint}"
    got = dout.numpy()
    nz = lens > 0
    assert np.all(got[~nz] == 0), what
    if nz.any():
        ref = oracle.attention_ragged(q[nz], widen(kb, dt), widen(vb, dt), offs[nz], lens[nz], NH, NKV, HD,
                                      n_threads=8)
        assert_close(got[nz], ref, what)
    assert ctx.check_device_error() == 0, what


@pytest.mark.parametrize("pos,kernel", [(0, 0), (200, 0), (1500, tmac_attn.TMAC_KERNEL_GROUP),
                                        (90, tmac_attn.TMAC_KERNEL_HEAD), (3000, 0)])
def test_layer_step_q8(ctx, pos, kernel):
    cap = pos + 20
    q, kn, vn = data(1000 + pos, NH * HD), data(1001 + pos, KVD), data(1002 + pos, KVD)
    kb = store(data(1003 + pos, (cap, KVD), 2), Q8)
    vb = store(data(1004 + pos, (cap, KVD), 2), Q8)
    dq, dkn, dvn = ctx.upload(q), ctx.upload(kn), ctx.upload(vn)
    dk, dv, dout = ctx.upload(kb), ctx.upload(vb), ctx.empty(NH * HD)
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, kernel)
    try:
        ctx.layer_attention(dq, dkn, dvn, dk, dv, dout, NH, NKV, HD, pos, cap, 1e6, kv_dtype=Q8)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, 0)
    qr, kr = oracle.rope(q, kn, NH, NKV, HD, pos, 1e6)
    kb_ref, vb_ref = kb.copy(), vb.copy()
    kb_ref[pos] = store(kr, Q8)[0]
    vb_ref[pos] = store(vn, Q8)[0]
    np.testing.assert_array_equal(dk.numpy(), kb_ref)
    np.testing.assert_array_equal(dv.numpy(), vb_ref)
    ref = oracle.attention(qr, widen(kb_ref, Q8), widen(vb_ref, Q8), NH, NKV, HD, pos)
    assert_close(dout.numpy(), ref, f"layer q8 pos={pos}")


@pytest.mark.parametrize("seed", range(12))
def test_layer_step_random_cases(ctx, seed):
    """Seeded random fused layer steps on every cache type: position (0, short
    or long), RoPE base, kernel choice (automatic, group, head, split-V head),
    MFMA or VALU decode, forced split length, and the position passed by value
    or in a device counter.  The cache rows are checked bit for bit and the
    output against the oracle's layer step."""
    rng = np.random.default_rng(2000 + seed)
    dt = ALL_DT[seed % len(ALL_DT)]
    pos = int(rng.choice([0, int(rng.integers(1, 64)), int(rng.integers(64, 5000))]))
    cap = pos + int(rng.integers(1, 40))
    base = float(rng.choice([1e4, 1e6]))
    kernel = int(rng.choice([tmac_attn.TMAC_KERNEL_AUTO, tmac_attn.TMAC_KERNEL_GROUP, tmac_attn.TMAC_KERNEL_HEAD,
                             tmac_attn.TMAC_KERNEL_HEADV]))
    mfma = int(rng.integers(0, 2))
    split_len = int(rng.choice([0, 0, 32, 256]))
    devpos = bool(rng.integers(0, 2))
    q, kn, vn = data(2100 + seed, NH * HD), data(2200 + seed, KVD), data(2300 + seed, KVD)
    kb = store(data(2400 + seed, (cap, KVD), 2), dt)
    vb = store(data(2500 + seed, (cap, KVD), 2), dt)
    dq, dkn, dvn = ctx.upload(q), ctx.upload(kn), ctx.upload(vn)
    dk, dv, dout = ctx.upload(kb), ctx.upload(vb), ctx.empty(NH * HD)
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, kernel)
    ctx.set_option(tmac_attn.TMAC_OPT_MFMA_DECODE, mfma)
    ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, split_len)
    try:
        if devpos:
            dpos = ctx.upload(np.array([pos], np.int32))
            ctx.layer_attention_devpos(dq, dkn, dvn, dk, dv, dout, NH, NKV, HD, dpos, cap, base, kv_dtype=dt)
        else:
            ctx.layer_attention(dq, dkn, dvn, dk, dv, dout, NH, NKV, HD, pos, cap, base, kv_dtype=dt)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, 0)
        ctx.set_option(tmac_attn.TMAC_OPT_MFMA_DECODE, 1)
        ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 0)
    what = (f"seed {seed}: dt={dt} pos={pos} cap={cap} base={base} kernel={kernel} mfma={mfma} "
            f"split={split_len} devpos={devpos}")
    qr, kr = oracle.rope(q, kn, NH, NKV, HD, pos, base)
    kb_ref, vb_ref = kb.copy(), vb.copy()
    kb_ref[pos] = store(kr, dt)[0]
    vb_ref[pos] = store(vn, dt)[0]
    np.testing.assert_array_equal(dk.numpy(), kb_ref, err_msg=what)
    np.testing.assert_array_equal(dv.numpy(), vb_ref, err_msg=what)
    ref = oracle.attention(qr, widen(kb_ref, dt), widen(vb_ref, dt), NH, NKV, HD, pos)
    assert_close(dout.numpy(), ref, what)
    assert ctx.check_device_error() == 0, what


def rows_of(x: np.ndarray, dt: int, rb: int) -> np.ndarray:
    """fp32 values -> stored cache rows of rb elements, for any number of kv heads."""
    flat = np.ascontiguousarray(x, np.float32).reshape(-1)
    if dt == Q8:
        return oracle.q8_kv_rows(flat.reshape(-1, HD)).reshape(-1, rb)
    # the 16-bit casts are elementwise: pad to whole 128-value rows for store()
    pad = np.concatenate([flat, np.zeros(-flat.size % KVD, np.float32)])
    return store(pad, dt).reshape(-1)[:flat.size].reshape(-1, rb)


def values_of(rows: np.ndarray, dt: int, width: int) -> np.ndarray:
    """Stored cache rows -> fp32 values [n, width], exactly."""
    flat = np.ascontiguousarray(rows).reshape(-1)
    if dt == Q8:
        return oracle.q8_kv_widen(flat.reshape(-1, oracle.Q8_HEAD_BYTES)).reshape(-1, width)
    pad = np.concatenate([flat, np.zeros(-flat.size % KVD, flat.dtype)])
    return widen(pad, dt).reshape(-1)[:flat.size].reshape(-1, width)


@pytest.mark.parametrize("dt", ALL_DT)
@pytest.mark.parametrize("mfma", [0, 1])
@pytest.mark.parametrize("pos,split_len", [(40, 64), (1500, 0), (333, 16)])
@pytest.mark.parametrize("g,kv", [(7, 2), (8, 1), (2, 2)])
def test_layer_step_reused_workspace(ctx, dt, mfma, pos, split_len, g, kv):
    """The layer step twice in a row with different data: the second call's
    split partials land on the first call's (every head of every split must be
    rewritten) and the output starts as NaN (every element must be written),
    one split (direct output) and several."""
    nh, kvd, cap = g * kv, kv * HD, pos + 20
    rb = kv * oracle.Q8_HEAD_BYTES if dt == Q8 else kvd
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, tmac_attn.TMAC_KERNEL_GROUP)
    ctx.set_option(tmac_attn.TMAC_OPT_MFMA_DECODE, mfma)
    ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, split_len)
    try:
        for call in range(2):
            s = 7000 + 10 * call + pos
            q, kn, vn = data(s, nh * HD), data(s + 1, kvd), data(s + 2, kvd)
            k_all, v_all = data(s + 3, (cap, kvd), 2), data(s + 4, (cap, kvd), 2)
            kb, vb = rows_of(k_all, dt, rb), rows_of(v_all, dt, rb)
            dq, dkn, dvn = ctx.upload(q), ctx.upload(kn), ctx.upload(vn)
            dk, dv = ctx.upload(kb), ctx.upload(vb)
            dout = ctx.upload(np.full(nh * HD, np.nan, np.float32))
            ctx.layer_attention(dq, dkn, dvn, dk, dv, dout, nh, kv, HD, pos, cap, 1e6, kv_dtype=dt)
            qr, kr = oracle.rope(q, kn, nh, kv, HD, pos, 1e6)
            kw, vw = values_of(kb, dt, kvd), values_of(vb, dt, kvd)
            kw[pos] = values_of(rows_of(kr, dt, rb), dt, kvd)[0]
            vw[pos] = values_of(rows_of(vn, dt, rb), dt, kvd)[0]
            np.testing.assert_array_equal(dk.numpy()[pos], rows_of(kr, dt, rb)[0])
            np.testing.assert_array_equal(dv.numpy()[pos], rows_of(vn, dt, rb)[0])
            ref = oracle.attention(qr, kw, vw, nh, kv, HD, pos)
            assert_close(dout.numpy(), ref, f"layer dt={dt} mfma={mfma} pos={pos} split={split_len} g={g} kv={kv} "
                                            f"call={call}")
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, 0)
        ctx.set_option(tmac_attn.TMAC_OPT_MFMA_DECODE, 1)
        ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 0)
    assert ctx.check_device_error() == 0


def test_graph_replay_q8(ctx):
    L, cap, S = 3, 64, 8
    rb = NKV * oracle.Q8_HEAD_BYTES
    kc, vc = ctx.upload(np.zeros((L, cap, rb), np.uint8)), ctx.upload(np.zeros((L, cap, rb), np.uint8))
    ref_k, ref_v = np.zeros((L, cap, rb), np.uint8), np.zeros((L, cap, rb), np.uint8)
    dq, dkn, dvn, dout = ctx.empty((L, NH * HD)), ctx.empty((L, KVD)), ctx.empty((L, KVD)), ctx.empty((L, NH * HD))
    pos = ctx.upload(np.zeros(1, np.int32))
    ctx.rope_prepare(HD, 1e6, cap)
    s = ctx.stream()
    ctx.step_begin(s)
    for layer in range(L):
        ctx.layer_attention_devpos(dq.at(layer * NH * HD), dkn.at(layer * KVD), dvn.at(layer * KVD),
                                   kc.at(layer * cap * rb), vc.at(layer * cap * rb), dout.at(layer * NH * HD),
                                   NH, NKV, HD, pos, cap, 1e6, stream=s, kv_dtype=Q8)
    ctx.pos_update(pos, 1, add=True, stream=s)
    g = ctx.step_end(s)
    try:
        for step in range(S):
            q, kn, vn = data(1100 + step, (L, NH * HD)), data(1200 + step, (L, KVD)), data(1300 + step, (L, KVD))
            dq.copy_from(q)
            dkn.copy_from(kn)
            dvn.copy_from(vn)
            ctx.graph_launch(g, s)
            ctx.synchronize(s)
            got = dout.numpy()
            for layer in range(L):
                qr, kr = oracle.rope(q[layer], kn[layer], NH, NKV, HD, step, 1e6)
                ref_k[layer, step] = store(kr, Q8)[0]
                ref_v[layer, step] = store(vn[layer], Q8)[0]
                ref = oracle.attention(qr, widen(ref_k[layer], Q8), widen(ref_v[layer], Q8), NH, NKV, HD, step)
                assert_close(got[layer], ref, f"q8 step {step} layer {layer}")
        np.testing.assert_array_equal(kc.numpy(), ref_k)
        np.testing.assert_array_equal(vc.numpy(), ref_v)
    finally:
        ctx.graph_destroy(g)
        ctx.destroy_stream(s)
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("dt", [tmac_attn.TMAC_KV_F32, tmac_attn.TMAC_KV_BF16, Q8])
def test_graph_replay_split_layer_step(ctx, dt):
    """A captured 3-layer step at long context (positions 1500.. read on the
    device), where every layer spreads its rows over many workgroups and a
    combine launch merges them; replayed with new inputs, each replay checked
    against the oracle, the cache rows it wrote bit for bit."""
    L, cap, P0, S = 3, 1600, 1500, 4
    rb = NKV * oracle.Q8_HEAD_BYTES if dt == Q8 else KVD
    ref_k = np.stack([rows_of(data(1500 + l, (cap, KVD), 2), dt, rb) for l in range(L)])
    ref_v = np.stack([rows_of(data(1600 + l, (cap, KVD), 2), dt, rb) for l in range(L)])
    kc, vc = ctx.upload(ref_k), ctx.upload(ref_v)
    dq, dkn, dvn, dout = ctx.empty((L, NH * HD)), ctx.empty((L, KVD)), ctx.empty((L, KVD)), ctx.empty((L, NH * HD))
    pos = ctx.upload(np.array([P0], np.int32))
    ctx.rope_prepare(HD, 1e6, cap)
    s = ctx.stream()
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, tmac_attn.TMAC_KERNEL_GROUP)
    try:
        def layer(i):
            ctx.layer_attention_devpos(dq.at(i * NH * HD), dkn.at(i * KVD), dvn.at(i * KVD), kc.at(i * cap * rb),
                                       vc.at(i * cap * rb), dout.at(i * NH * HD), NH, NKV, HD, pos, cap, 1e6,
                                       stream=s, kv_dtype=dt)
        n_splits = ctx.query_split(1, cap, NH, NKV)[1]
        assert n_splits > 8, n_splits
        for i in range(L):  # sizes the split workspace outside capture (and writes row P0; rewritten below)
            layer(i)
        ctx.synchronize(s)
        ctx.step_begin(s)
        for i in range(L):
            layer(i)
        ctx.pos_update(pos, 1, add=True, stream=s)
        g = ctx.step_end(s)
        try:
            for step in range(S):
                p = P0 + step
                q, kn, vn = data(1700 + step, (L, NH * HD)), data(1800 + step, (L, KVD)), data(1900 + step, (L, KVD))
                dq.copy_from(q)
                dkn.copy_from(kn)
                dvn.copy_from(vn)
                ctx.graph_launch(g, s)
                ctx.synchronize(s)
                got = dout.numpy()
                for l in range(L):
                    qr, kr = oracle.rope(q[l], kn[l], NH, NKV, HD, p, 1e6)
                    ref_k[l, p] = rows_of(kr, dt, rb)[0]
                    ref_v[l, p] = rows_of(vn[l], dt, rb)[0]
                    ref = oracle.attention(qr, values_of(ref_k[l], dt, KVD), values_of(ref_v[l], dt, KVD), NH, NKV,
                                           HD, p)
                    assert_close(got[l], ref, f"dt={dt} pos={p} layer={l}")
            np.testing.assert_array_equal(kc.numpy(), ref_k)
            np.testing.assert_array_equal(vc.numpy(), ref_v)
            assert int(pos.numpy()[0]) == P0 + S
        finally:
            ctx.graph_destroy(g)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, 0)
        ctx.destroy_stream(s)
    assert ctx.check_device_error() == 0


def test_q8_storage_error_against_fp32_cache(ctx):
    """Not a parity bar: what storing the cache as Q8_0 does to the output,
    against the fp32 cache (N(0,1) data, 4096 rows)."""
    n_seq, n_pos = 4, 4096
    q = data(1400, (n_seq, NH * HD))
    k, v = data(1401, (n_seq * n_pos, KVD)), data(1402, (n_seq * n_pos, KVD))
    dq, dout = ctx.upload(q), ctx.empty((n_seq, NH * HD))
    dk, dv = ctx.upload(store(k, Q8)), ctx.upload(store(v, Q8))
    ctx.decode_batched(dq, dk, dv, dout, n_seq, NH, NKV, HD, n_pos, n_pos, kv_dtype=Q8)
    offs = np.arange(n_seq, dtype=np.int64) * n_pos
    ref32 = oracle.attention_ragged(q, k, v, offs, np.full(n_seq, n_pos, np.int32), NH, NKV, HD, n_threads=8)
    err = float(np.abs(dout.numpy() - ref32).max())
    print(f"q8_0 cache: max |out_q8 - out_f32| = {err:.3e}")
    assert err < 2e-2


# ---- paged caches ---------------------------------------------------------------------------------

def build_pool(rows_per_seq, dt, n_pages, rng, shared_prefix_pages=0):
    """Scatters each sequence's stored rows into a pool of n_pages pages in a
    random page order.  Sequence 1 may share sequence 0's first
    `shared_prefix_pages` pages (same physical pages; the rows must match).
    Unused pages hold garbage.  Returns pool [n_pages * 16, row], table."""
    n_seq = len(rows_per_seq)
    max_pages = max(1, max((r.shape[0] + PR - 1) // PR for r in rows_per_seq))
    width = rows_per_seq[0].shape[1]
    pool = rng.integers(0, 256, (n_pages * PR * width * rows_per_seq[0].itemsize,), np.uint8).view(
        rows_per_seq[0].dtype).reshape(n_pages * PR, width)
    if dt == tmac_attn.TMAC_KV_F32:  # garbage that is still a float (no NaN in unused rows of used pages)
        pool[:] = rng.standard_normal(pool.shape).astype(np.float32) * 1e3
    perm = rng.permutation(n_pages)
    table = np.full((n_seq, max_pages), -1, np.int32)  # entries past a sequence's pages are never read
    nxt = 0
    for s, r in enumerate(rows_per_seq):
        n_p = (r.shape[0] + PR - 1) // PR
        for j in range(n_p):
            if s == 1 and j < shared_prefix_pages:
                table[s, j] = table[0, j]
                continue
            table[s, j] = perm[nxt]
            nxt += 1
            seg = r[j * PR:(j + 1) * PR]
            pool[table[s, j] * PR:table[s, j] * PR + seg.shape[0]] = seg
    assert nxt <= n_pages
    table[table < 0] = 0
    return pool, table


@pytest.mark.parametrize("dt", ALL_DT)
@pytest.mark.parametrize("hint", [0, 1])
def test_decode_paged(ctx, dt, hint):
    rng = np.random.default_rng(50 + dt)
    lens = np.array([1, 0, 15, 16, 17, 1000, 4000, 33, 2048], np.int32)
    n_seq = lens.size
    k_rows = [store(data(60 + s, (max(int(lens[s]), 1), KVD), 2), dt)[:lens[s]] for s in range(n_seq)]
    v_rows = [store(data(90 + s, (max(int(lens[s]), 1), KVD), 2), dt)[:lens[s]] for s in range(n_seq)]
    n_pages = int(sum((l + PR - 1) // PR for l in lens)) + 11
    kp, table = build_pool(k_rows, dt, n_pages, np.random.default_rng(7))
    vp, table_v = build_pool(v_rows, dt, n_pages, np.random.default_rng(7))
    assert np.array_equal(table, table_v)
    q = data(300 + dt, (n_seq, NH * HD))
    dq, dk, dv, dt_, dl = ctx.upload(q), ctx.upload(kp), ctx.upload(vp), ctx.upload(table), ctx.upload(lens)
    dout = ctx.empty((n_seq, NH * HD))
    max_len = int(lens.max())
    ctx.decode_paged(dq, dk, dv, n_pages, dt_, table.shape[1], dl, dout, n_seq, NH, NKV, HD, max_len,
                     total_rows=int(lens.sum()) if hint else 0, kv_dtype=dt)
    got = dout.numpy()
    nz = lens > 0
    kw = np.concatenate([widen(r, dt) for r in k_rows if r.shape[0]])
    vw = np.concatenate([widen(r, dt) for r in v_rows if r.shape[0]])
    offs = np.concatenate([[0], np.cumsum(lens[nz][:-1])]).astype(np.int64)
    ref = oracle.attention_ragged(q[nz], kw, vw, offs, lens[nz], NH, NKV, HD, n_threads=8)
    assert np.all(got[~nz] == 0)
    assert_close(got[nz], ref, f"paged dt={dt} hint={hint}")
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("dt", [tmac_attn.TMAC_KV_BF16, Q8])
def test_decode_paged_long_splits(ctx, dt):
    """Paged MFMA decode with one split per sequence: every wave walks many
    pages through the tile loop's steady state and drain (lengths as in the
    contiguous long-split test, plus one page exactly)."""
    lens = np.array([336, 512, 695, 2085, 16], np.int32)
    n_seq = lens.size
    k_rows = [store(data(860 + s, (int(lens[s]), KVD), 2), dt) for s in range(n_seq)]
    v_rows = [store(data(870 + s, (int(lens[s]), KVD), 2), dt) for s in range(n_seq)]
    n_pages = int(sum((l + PR - 1) // PR for l in lens)) + 5
    kp, table = build_pool(k_rows, dt, n_pages, np.random.default_rng(11))
    vp, _ = build_pool(v_rows, dt, n_pages, np.random.default_rng(11))
    q = data(880 + dt, (n_seq, NH * HD))
    dq, dk, dv, dt_, dl = ctx.upload(q), ctx.upload(kp), ctx.upload(vp), ctx.upload(table), ctx.upload(lens)
    dout = ctx.empty((n_seq, NH * HD))
    ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 4096)
    try:
        ctx.decode_paged(dq, dk, dv, n_pages, dt_, table.shape[1], dl, dout, n_seq, NH, NKV, HD, int(lens.max()),
                         kv_dtype=dt)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 0)
    kw = np.concatenate([widen(r, dt) for r in k_rows])
    vw = np.concatenate([widen(r, dt) for r in v_rows])
    offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
    ref = oracle.attention_ragged(q, kw, vw, offs, lens, NH, NKV, HD, n_threads=8)
    assert_close(dout.numpy(), ref, f"paged long splits dt={dt}")
    assert ctx.check_device_error() == 0


def test_decode_paged_shared_prefix_and_splits(ctx):
    """Two sequences sharing their first 40 pages; a forced short split length
    so that every sequence spans many workgroups and the combine kernel runs."""
    dt = tmac_attn.TMAC_KV_F32
    base_k, base_v = data(400, (1500, KVD)), data(401, (1500, KVD))
    lens = np.array([1500, 1200, 700], np.int32)
    k_rows = [base_k, np.concatenate([base_k[:640], data(402, (560, KVD))]), data(403, (700, KVD))]
    v_rows = [base_v, np.concatenate([base_v[:640], data(404, (560, KVD))]), data(405, (700, KVD))]
    n_pages = 300
    kp, table = build_pool(k_rows, dt, n_pages, np.random.default_rng(9), shared_prefix_pages=40)
    vp, table_v = build_pool(v_rows, dt, n_pages, np.random.default_rng(9), shared_prefix_pages=40)
    assert np.array_equal(table, table_v) and np.array_equal(table[0, :40], table[1, :40])
    q = data(406, (3, NH * HD))
    dq, dk, dv, dtab, dl = ctx.upload(q), ctx.upload(kp), ctx.upload(vp), ctx.upload(table), ctx.upload(lens)
    dout = ctx.empty((3, NH * HD))
    ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 64)
    try:
        ctx.decode_paged(dq, dk, dv, n_pages, dtab, table.shape[1], dl, dout, 3, NH, NKV, HD, 1500)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 0)
    offs = np.array([0, 1500, 2700], np.int64)
    ref = oracle.attention_ragged(q, np.concatenate(k_rows), np.concatenate(v_rows), offs, lens, NH, NKV, HD,
                                  n_threads=8)
    assert_close(dout.numpy(), ref, "shared prefix")
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("dt", ALL_DT)
@pytest.mark.parametrize("mfma", [0, 1])
def test_split_merge_repeated_calls(ctx, dt, mfma):
    """Many splits per sequence (forced 64-row splits) merged by the combine
    launch: ragged, paged and batched decode, each called three times in a
    row with new queries over the same split workspace."""
    lens = np.array([1, 0, 700, 3001, 64, 65, 1500], np.int32)
    n_seq = lens.size
    offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
    rows = int(lens.sum())
    kb, vb = store(data(2100 + dt, (rows, KVD), 2), dt), store(data(2101 + dt, (rows, KVD), 2), dt)
    kw, vw = widen(kb, dt), widen(vb, dt)
    k_rows = [kb[o:o + n] for o, n in zip(offs, lens)]
    v_rows = [vb[o:o + n] for o, n in zip(offs, lens)]
    n_pages = int(sum((l + PR - 1) // PR for l in lens)) + 5
    kp, table = build_pool(k_rows, dt, n_pages, np.random.default_rng(21))
    vp, _ = build_pool(v_rows, dt, n_pages, np.random.default_rng(21))
    dk, dv, doffs, dlens = ctx.upload(kb), ctx.upload(vb), ctx.upload(offs), ctx.upload(lens)
    dkp, dvp, dtab = ctx.upload(kp), ctx.upload(vp), ctx.upload(table)
    dout = ctx.empty((n_seq, NH * HD))
    nz = lens > 0
    ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 64)
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, tmac_attn.TMAC_KERNEL_GROUP)
    ctx.set_option(tmac_attn.TMAC_OPT_MFMA_DECODE, mfma)
    try:
        for call in range(3):
            q = data(2200 + 10 * dt + call, (n_seq, NH * HD))
            dq = ctx.upload(q)
            ref = oracle.attention_ragged(q[nz], kw, vw, offs[nz], lens[nz], NH, NKV, HD, n_threads=8)
            ctx.decode_ragged(dq, dk, dv, doffs, dlens, dout, n_seq, NH, NKV, HD, int(lens.max()), kv_dtype=dt)
            got = dout.numpy()
            assert np.all(got[~nz] == 0)
            assert_close(got[nz], ref, f"ragged dt={dt} mfma={mfma} call={call}")
            ctx.decode_paged(dq, dkp, dvp, n_pages, dtab, table.shape[1], dlens, dout, n_seq, NH, NKV, HD,
                             int(lens.max()), kv_dtype=dt)
            got = dout.numpy()
            assert np.all(got[~nz] == 0)
            assert_close(got[nz], ref, f"paged dt={dt} mfma={mfma} call={call}")
            # batched: the first 3 x 700 rows as three sequences
            ctx.decode_batched(dq, dk, dv, dout, 3, NH, NKV, HD, 700, 700, kv_dtype=dt)
            ref_b = oracle.attention_ragged(q[:3], kw, vw, np.array([0, 700, 1400], np.int64),
                                            np.full(3, 700, np.int32), NH, NKV, HD, n_threads=8)
            assert_close(dout.numpy()[:3], ref_b, f"batched dt={dt} mfma={mfma} call={call}")
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 0)
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, 0)
        ctx.set_option(tmac_attn.TMAC_OPT_MFMA_DECODE, 1)
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("dt", [tmac_attn.TMAC_KV_F32, Q8])
def test_split_merge_graph_replay(ctx, dt):
    """A captured ragged decode with many splits per sequence (decode and
    combine launches), replayed with new queries, with eager calls of the same
    shape between the replays."""
    lens = np.array([3001, 64, 1500, 9], np.int32)
    n_seq = lens.size
    offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
    rows = int(lens.sum())
    kb, vb = store(data(2300, (rows, KVD), 2), dt), store(data(2301, (rows, KVD), 2), dt)
    kw, vw = widen(kb, dt), widen(vb, dt)
    dk, dv, doffs, dlens = ctx.upload(kb), ctx.upload(vb), ctx.upload(offs), ctx.upload(lens)
    dq, dout = ctx.empty((n_seq, NH * HD)), ctx.empty((n_seq, NH * HD))
    s = ctx.stream()
    ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 64)
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, tmac_attn.TMAC_KERNEL_GROUP)
    try:
        ctx.decode_ragged(dq, dk, dv, doffs, dlens, dout, n_seq, NH, NKV, HD, int(lens.max()), stream=s,
                          kv_dtype=dt)  # sizes the split workspace outside capture
        ctx.synchronize(s)
        ctx.step_begin(s)
        ctx.decode_ragged(dq, dk, dv, doffs, dlens, dout, n_seq, NH, NKV, HD, int(lens.max()), stream=s,
                          kv_dtype=dt)
        g = ctx.step_end(s)
        try:
            for rep in range(4):
                for eager in (False, True):
                    q = data(2400 + 2 * rep + eager, (n_seq, NH * HD))
                    dq.copy_from(q)
                    if eager:
                        ctx.decode_ragged(dq, dk, dv, doffs, dlens, dout, n_seq, NH, NKV, HD, int(lens.max()),
                                          stream=s, kv_dtype=dt)
                    else:
                        ctx.graph_launch(g, s)
                    ctx.synchronize(s)
                    ref = oracle.attention_ragged(q, kw, vw, offs, lens, NH, NKV, HD, n_threads=8)
                    assert_close(dout.numpy(), ref, f"dt={dt} replay={rep} eager={eager}")
        finally:
            ctx.graph_destroy(g)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 0)
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, 0)
        ctx.destroy_stream(s)
    assert ctx.check_device_error() == 0


def test_decode_paged_bad_page_is_reported(ctx):
    """A block-table entry outside the pool is clamped into it by the kernel
    (so every access stays in bounds) and reported through the error word."""
    n_pages = 8
    kp = np.zeros((n_pages * PR, KVD), np.float32)
    table = np.array([[0, 1, n_pages + 5]], np.int32)
    lens = np.array([40], np.int32)
    dq, dout = ctx.upload(data(500, (1, NH * HD))), ctx.empty((1, NH * HD))
    dk, dtab, dl = ctx.upload(kp), ctx.upload(table), ctx.upload(lens)
    ctx.decode_paged(dq, dk, dk, n_pages, dtab, 3, dl, dout, 1, NH, NKV, HD, 48)
    assert ctx.check_device_error() == tmac_attn.TMAC_ERR_DEVICE_FAULT
    assert ctx.check_device_error() == 0  # cleared


def test_decode_paged_rejects(ctx):
    d = ctx.empty(4096)
    t = ctx.upload(np.zeros((1, 2), np.int32))
    ok = dict(n_seq=1, n_head=NH, n_kv_head=NKV, head_dim=HD)
    assert ctx.decode_paged(d, d, d, 4, t, 2, t, d, max_len=33, check=False, **ok) == tmac_attn.TMAC_ERR_INVALID_ARG
    assert ctx.decode_paged(d, d, d, 0, t, 2, t, d, max_len=8, check=False, **ok) == tmac_attn.TMAC_ERR_INVALID_ARG
    assert ctx.decode_paged(d, d, d, 4, t, 2, t, d, max_len=8, kv_dtype=7, check=False, **ok) == \
        tmac_attn.TMAC_ERR_INVALID_ARG
    assert ctx.decode_paged(d, d, None, 4, t, 2, t, d, max_len=8, check=False, **ok) == \
        tmac_attn.TMAC_ERR_NULL_POINTER


@pytest.mark.parametrize("dt", ALL_DT)
def test_layer_paged_batch(ctx, dt):
    """One batched layer step: sequences at different positions (one at 0, one
    at a page boundary), RoPE + the new row written into its page + attention."""
    positions = np.array([0, 15, 16, 300, 1999, 47], np.int32)
    n_seq = positions.size
    max_len = int(positions.max()) + 1
    k_rows = [store(data(600 + s, (int(p) + 1, KVD), 2), dt) for s, p in enumerate(positions)]
    v_rows = [store(data(700 + s, (int(p) + 1, KVD), 2), dt) for s, p in enumerate(positions)]
    n_pages = int(sum((p + PR) // PR for p in positions)) + 5
    kp, table = build_pool(k_rows, dt, n_pages, np.random.default_rng(13))
    vp, _ = build_pool(v_rows, dt, n_pages, np.random.default_rng(13))
    q, kn, vn = data(800 + dt, (n_seq, NH * HD)), data(801 + dt, (n_seq, KVD)), data(802 + dt, (n_seq, KVD))
    dq, dkn, dvn = ctx.upload(q), ctx.upload(kn), ctx.upload(vn)
    dk, dv, dtab, dpos = ctx.upload(kp), ctx.upload(vp), ctx.upload(table), ctx.upload(positions)
    dout = ctx.empty((n_seq, NH * HD))
    ctx.layer_attention_paged(dq, dkn, dvn, dk, dv, n_pages, dtab, table.shape[1], dpos, dout, n_seq, NH, NKV,
                              HD, max_len, 1e6, kv_dtype=dt)
    got, kp_got, vp_got = dout.numpy(), dk.numpy(), dv.numpy()
    kp_ref, vp_ref = kp.copy(), vp.copy()
    for s, p in enumerate(positions):
        qr, kr = oracle.rope(q[s], kn[s], NH, NKV, HD, int(p), 1e6)
        row = table[s, p // PR] * PR + p % PR
        kp_ref[row] = store(kr, dt)[0]
        vp_ref[row] = store(vn[s], dt)[0]
        rows = np.array([table[s, r // PR] * PR + r % PR for r in range(p + 1)])
        ref = oracle.attention(qr, widen(kp_ref[rows], dt), widen(vp_ref[rows], dt), NH, NKV, HD, int(p))
        assert_close(got[s], ref, f"paged layer dt={dt} seq {s} pos {p}")
    np.testing.assert_array_equal(kp_got, kp_ref)
    np.testing.assert_array_equal(vp_got, vp_ref)
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("dt", [tmac_attn.TMAC_KV_F32, Q8])
def test_layer_paged_graph_replay(ctx, dt):
    """A captured batched step replayed for 6 steps; the host advances the
    device-side positions between replays (sequences start at different
    positions and cross page boundaries)."""
    n_seq, S = 3, 6
    start = np.array([13, 0, 30], np.int32)
    max_len = 64
    max_pages = max_len // PR
    n_pages = n_seq * max_pages + 2
    table = (np.random.default_rng(3).permutation(n_pages)[:n_seq * max_pages]).reshape(n_seq, max_pages)
    table = table.astype(np.int32)
    width = store(np.zeros((1, KVD), np.float32), dt).shape[1]
    sdt = store(np.zeros((1, KVD), np.float32), dt).dtype
    kp = np.zeros((n_pages * PR, width), sdt)
    vp = np.zeros((n_pages * PR, width), sdt)
    for s in range(n_seq):  # history rows 0..start-1
        for r in range(int(start[s])):
            kp[table[s, r // PR] * PR + r % PR] = store(data(900 + 100 * s + r, (1, KVD)), dt)[0]
            vp[table[s, r // PR] * PR + r % PR] = store(data(950 + 100 * s + r, (1, KVD)), dt)[0]
    dk, dv, dtab = ctx.upload(kp), ctx.upload(vp), ctx.upload(table)
    dpos = ctx.upload(start)
    dq, dkn, dvn = ctx.empty((n_seq, NH * HD)), ctx.empty((n_seq, KVD)), ctx.empty((n_seq, KVD))
    dout = ctx.empty((n_seq, NH * HD))
    args = (dq, dkn, dvn, dk, dv, n_pages, dtab, max_pages, dpos, dout, n_seq, NH, NKV, HD, max_len, 1e6)
    dq.copy_from(np.zeros((n_seq, NH * HD), np.float32))
    dkn.copy_from(np.zeros((n_seq, KVD), np.float32))
    dvn.copy_from(np.zeros((n_seq, KVD), np.float32))
    ctx.rope_prepare(HD, 1e6, max_len)
    s_ = ctx.stream()
    ctx.step_begin(s_)
    ctx.layer_attention_paged(*args, stream=s_, kv_dtype=dt)
    g = ctx.step_end(s_)
    kp_ref, vp_ref = kp.copy(), vp.copy()
    try:
        for step in range(S):
            pos = start + step
            q, kn, vn = data(1500 + step, (n_seq, NH * HD)), data(1600 + step, (n_seq, KVD)), data(1700 + step,
                                                                                                  (n_seq, KVD))
            dq.copy_from(q)
            dkn.copy_from(kn)
            dvn.copy_from(vn)
            dpos.copy_from(pos.astype(np.int32))
            ctx.graph_launch(g, s_)
            ctx.synchronize(s_)
            got = dout.numpy()
            for s in range(n_seq):
                p = int(pos[s])
                qr, kr = oracle.rope(q[s], kn[s], NH, NKV, HD, p, 1e6)
                row = table[s, p // PR] * PR + p % PR
                kp_ref[row] = store(kr, dt)[0]
                vp_ref[row] = store(vn[s], dt)[0]
                rows = np.array([table[s, r // PR] * PR + r % PR for r in range(p + 1)])
                ref = oracle.attention(qr, widen(kp_ref[rows], dt), widen(vp_ref[rows], dt), NH, NKV, HD, p)
                assert_close(got[s], ref, f"replay dt={dt} step {step} seq {s}")
        np.testing.assert_array_equal(dk.numpy(), kp_ref)
        np.testing.assert_array_equal(dv.numpy(), vp_ref)
    finally:
        ctx.graph_destroy(g)
        ctx.destroy_stream(s_)
    assert ctx.check_device_error() == 0


def test_layer_paged_position_errors(ctx):
    """A position at or past 16 * max_pages is skipped and reported (bit 0);
    one past max_len gives NaN output (bit 1); the other sequences are exact."""
    n_pages, max_pages = 12, 4
    kp = np.zeros((n_pages * PR, KVD), np.float32)
    table = np.arange(12, dtype=np.int32).reshape(3, 4)
    positions = np.array([5, 64, 40], np.int32)  # 64 = 16 * max_pages: outside; 40 >= max_len 32
    q, kn, vn = data(1800, (3, NH * HD)), data(1801, (3, KVD)), data(1802, (3, KVD))
    dq, dkn, dvn, dk, dv = ctx.upload(q), ctx.upload(kn), ctx.upload(vn), ctx.upload(kp), ctx.upload(kp)
    dtab, dpos, dout = ctx.upload(table), ctx.upload(positions), ctx.empty((3, NH * HD))
    ctx.layer_attention_paged(dq, dkn, dvn, dk, dv, n_pages, dtab, max_pages, dpos, dout, 3, NH, NKV, HD, 32, 1e6)
    got = dout.numpy()
    assert ctx.check_device_error() == tmac_attn.TMAC_ERR_DEVICE_FAULT
    assert np.all(np.isnan(got[2]))
    qr, kr = oracle.rope(q[0], kn[0], NH, NKV, HD, 5, 1e6)
    kref, vref = np.zeros((6, KVD), np.float32), np.zeros((6, KVD), np.float32)
    kref[5], vref[5] = kr, vn[0]
    assert_close(got[0], oracle.attention(qr, kref, vref, NH, NKV, HD, 5), "valid sequence")


@pytest.mark.parametrize("g,kv", [(1, 1), (2, 2), (4, 4), (8, 1)])
def test_decode_q8_mfma_shapes(ctx, g, kv):
    """Q8_0 decode (MFMA kernel) at other GQA shapes, ragged, with widely
    varying row magnitudes (per-block scales from 2^-4 to 2^4)."""
    nh, kvd = g * kv, kv * HD
    lens = np.array([513, 1, 40, 1500], np.int32)
    offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
    rows = int(lens.sum())
    q = data(1900 + g + kv, (lens.size, nh * HD))
    kb = oracle.q8_kv_rows(data(1901 + g + kv, (rows, kvd), 4)).reshape(rows, -1)
    vb = oracle.q8_kv_rows(data(1902 + g + kv, (rows, kvd), 4)).reshape(rows, -1)
    dq, dk, dv = ctx.upload(q), ctx.upload(kb), ctx.upload(vb)
    doffs, dlens, dout = ctx.upload(offs), ctx.upload(lens), ctx.empty((lens.size, nh * HD))
    ctx.decode_ragged(dq, dk, dv, doffs, dlens, dout, lens.size, nh, kv, HD, int(lens.max()), kv_dtype=Q8)
    kw = oracle.q8_kv_widen(kb).reshape(rows, kvd)
    vw = oracle.q8_kv_widen(vb).reshape(rows, kvd)
    ref = oracle.attention_ragged(q, kw, vw, offs, lens, nh, kv, HD, n_threads=8)
    assert_close(dout.numpy(), ref, f"q8 ragged g={g} kv={kv}")
    assert ctx.check_device_error() == 0
