"""GPU parity of the 16-bit KV cache paths (tmac_*_kv with TMAC_KV_BF16 /
TMAC_KV_F16, tmac_kv_convert).

Contract: a 16-bit cache is read and widened exactly to fp32, so every output
must equal the oracle (tmac_gguf.cpp:1093-1128) run on the widened cache within
the fp32 tolerance |gpu - ref| <= 2e-5 + 1e-4 |ref|.  The layer step stores the
rotated k and v_new rounded to nearest even in the cache type; that row must
match the oracle's RoPE (tmac_gguf.cpp:990-1016) rounded the same way bit for
bit.  The conversion kernel is checked bit for bit against numpy.  How far a
16-bit cache moves the result from the fp32 cache is measured, not a parity
bar (last test).
"""
import numpy as np
import pytest

import oracle
import tmac_attn
from conftest import assert_close

pytestmark = pytest.mark.gpu
NH, NKV, HD = 14, 2, 64
KVD = NKV * HD
DTYPES = [tmac_attn.TMAC_KV_BF16, tmac_attn.TMAC_KV_F16]


def to16(x: np.ndarray, dt: int) -> np.ndarray:
    """fp32 -> 16-bit storage bits (uint16), round to nearest even."""
    x = np.ascontiguousarray(x, np.float32)
    if dt == tmac_attn.TMAC_KV_F16:
        return x.astype(np.float16).view(np.uint16)
    u = x.view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def widen(bits: np.ndarray, dt: int) -> np.ndarray:
    bits = np.ascontiguousarray(bits, np.uint16)
    if dt == tmac_attn.TMAC_KV_F16:
        return bits.view(np.float16).astype(np.float32)
    return (bits.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("dt", DTYPES)
def test_kv_convert_bit_exact(ctx, dt):
    rng = np.random.default_rng(70 + dt)
    x = (rng.standard_normal(5000) * np.exp(rng.uniform(-20, 20, 5000))).astype(np.float32)
    x[:4] = [0.0, -0.0, 65504.0, 1e-8]
    if dt == tmac_attn.TMAC_KV_F16:  # beyond the fp16 range both sides give inf; keep the warning out
        x = np.clip(x, -6e4, 6e4)
    dx, dy = ctx.upload(x), ctx.empty(x.size, np.uint16)
    ctx.kv_convert(dt, dx, dy, x.size)
    np.testing.assert_array_equal(dy.numpy(), to16(x, dt))


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("n_seq,n_pos,kernel", [(3, 300, tmac_attn.TMAC_KERNEL_AUTO), (2, 2000, 0),
                                                (8, 4096, 0), (1, 700, tmac_attn.TMAC_KERNEL_HEAD),
                                                (2, 77, tmac_attn.TMAC_KERNEL_GROUP)])
def test_decode_batched_16bit(ctx, dt, n_seq, n_pos, kernel):
    q = oracle.normal(800 + n_pos, (n_seq, NH * HD))
    kb = to16(oracle.normal(801 + n_pos, (n_seq, n_pos, KVD)), dt)
    vb = to16(oracle.normal(802 + n_pos, (n_seq, n_pos, KVD)), dt)
    dq, dk, dv, dout = ctx.upload(q), ctx.upload(kb), ctx.upload(vb), ctx.empty((n_seq, NH * HD))
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, kernel)
    try:
        ctx.decode_batched(dq, dk, dv, dout, n_seq, NH, NKV, HD, n_pos, n_pos, kv_dtype=dt)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, 0)
    kw, vw = widen(kb, dt), widen(vb, dt)
    offs = np.arange(n_seq, dtype=np.int64) * n_pos
    lens = np.full(n_seq, n_pos, np.int32)
    ref = oracle.attention_ragged(q, kw.reshape(-1, KVD), vw.reshape(-1, KVD), offs, lens, NH, NKV, HD,
                                  n_threads=8)
    assert_close(dout.numpy(), ref, f"batched dt={dt} {n_seq}x{n_pos}")


@pytest.mark.parametrize("dt", DTYPES)
def test_decode_ragged_16bit(ctx, dt):
    lens = np.array([1, 0, 513, 4000, 37, 2048, 3], np.int32)
    n_seq = lens.size
    offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64) + 5  # unaligned starts
    rows = int(offs[-1] + lens[-1])
    q = oracle.normal(900, (n_seq, NH * HD))
    kb = to16(oracle.normal(901, (rows, KVD)), dt)
    vb = to16(oracle.normal(902, (rows, KVD)), dt)
    dq, dk, dv = ctx.upload(q), ctx.upload(kb), ctx.upload(vb)
    doffs, dlens, dout = ctx.upload(offs), ctx.upload(lens), ctx.empty((n_seq, NH * HD))
    for hint in (0, int(lens.sum())):
        ctx.decode_ragged(dq, dk, dv, doffs, dlens, dout, n_seq, NH, NKV, HD, int(lens.max()), hint, kv_dtype=dt)
        nz = lens > 0
        ref = oracle.attention_ragged(q[nz], widen(kb, dt), widen(vb, dt), offs[nz], lens[nz], NH, NKV, HD,
                                      n_threads=8)
        got = dout.numpy()
        assert np.all(got[~nz] == 0)  # an empty sequence is a zero output
        assert_close(got[nz], ref, f"ragged dt={dt} hint={hint}")
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("pos,kernel", [(0, 0), (200, 0), (1500, tmac_attn.TMAC_KERNEL_GROUP),
                                        (90, tmac_attn.TMAC_KERNEL_HEAD)])
def test_layer_step_16bit(ctx, dt, pos, kernel):
    cap = pos + 20
    q = oracle.normal(1000 + pos, NH * HD)
    kn = oracle.normal(1001 + pos, KVD)
    vn = oracle.normal(1002 + pos, KVD)
    kb = to16(oracle.normal(1003 + pos, (cap, KVD)), dt)
    vb = to16(oracle.normal(1004 + pos, (cap, KVD)), dt)
    dq, dkn, dvn = ctx.upload(q), ctx.upload(kn), ctx.upload(vn)
    dk, dv, dout = ctx.upload(kb), ctx.upload(vb), ctx.empty(NH * HD)
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, kernel)
    try:
        ctx.layer_attention(dq, dkn, dvn, dk, dv, dout, NH, NKV, HD, pos, cap, 1e6, kv_dtype=dt)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, 0)
    qr, kr = oracle.rope(q, kn, NH, NKV, HD, pos, 1e6)
    kb_ref, vb_ref = kb.copy(), vb.copy()
    kb_ref[pos] = to16(kr, dt)
    vb_ref[pos] = to16(vn, dt)
    np.testing.assert_array_equal(dk.numpy(), kb_ref)
    np.testing.assert_array_equal(dv.numpy(), vb_ref)
    ref = oracle.attention(qr, widen(kb_ref, dt), widen(vb_ref, dt), NH, NKV, HD, pos)
    assert_close(dout.numpy(), ref, f"layer dt={dt} pos={pos}")


@pytest.mark.parametrize("dt", DTYPES)
def test_graph_replay_16bit(ctx, dt):
    """A captured 3-layer step with the position on the device, replayed for
    positions 0..7 on a bf16/fp16 cache, against the oracle step by step."""
    L, cap, S = 3, 64, 8
    kc = ctx.upload(np.zeros((L, cap, KVD), np.uint16))
    vc = ctx.upload(np.zeros((L, cap, KVD), np.uint16))
    ref_k = np.zeros((L, cap, KVD), np.uint16)
    ref_v = np.zeros((L, cap, KVD), np.uint16)
    dq, dkn, dvn, dout = ctx.empty((L, NH * HD)), ctx.empty((L, KVD)), ctx.empty((L, KVD)), ctx.empty((L, NH * HD))
    pos = ctx.upload(np.zeros(1, np.int32))
    ctx.rope_prepare(HD, 1e6, cap)
    s = ctx.stream()
    ctx.step_begin(s)
    for layer in range(L):
        ctx.layer_attention_devpos(dq.at(layer * NH * HD), dkn.at(layer * KVD), dvn.at(layer * KVD),
                                   kc.at(layer * cap * KVD), vc.at(layer * cap * KVD), dout.at(layer * NH * HD),
                                   NH, NKV, HD, pos, cap, 1e6, stream=s, kv_dtype=dt)
    ctx.pos_update(pos, 1, add=True, stream=s)
    g = ctx.step_end(s)
    try:
        for step in range(S):
            q = oracle.normal(1100 + step, (L, NH * HD))
            kn = oracle.normal(1200 + step, (L, KVD))
            vn = oracle.normal(1300 + step, (L, KVD))
            dq.copy_from(q)
            dkn.copy_from(kn)
            dvn.copy_from(vn)
            ctx.graph_launch(g, s)
            ctx.synchronize(s)
            got = dout.numpy()
            for layer in range(L):
                qr, kr = oracle.rope(q[layer], kn[layer], NH, NKV, HD, step, 1e6)
                ref_k[layer, step] = to16(kr, dt)
                ref_v[layer, step] = to16(vn[layer], dt)
                ref = oracle.attention(qr, widen(ref_k[layer], dt), widen(ref_v[layer], dt), NH, NKV, HD, step)
                assert_close(got[layer], ref, f"dt={dt} step {step} layer {layer}")
        np.testing.assert_array_equal(kc.numpy(), ref_k)
        np.testing.assert_array_equal(vc.numpy(), ref_v)
    finally:
        ctx.graph_destroy(g)
        ctx.destroy_stream(s)
    assert ctx.check_device_error() == 0


def test_rejects_bad_kv_dtype(ctx):
    d = ctx.empty(NH * HD * 4)
    assert ctx.decode_batched(d, d, d, d, 1, NH, NKV, HD, 2, 2, kv_dtype=4, check=False) == \
        tmac_attn.TMAC_ERR_INVALID_ARG
    assert ctx.kv_convert(tmac_attn.TMAC_KV_F32, d, d, 4, check=False) == tmac_attn.TMAC_ERR_INVALID_ARG


@pytest.mark.parametrize("dt", DTYPES)
def test_16bit_storage_error_against_fp32_cache(ctx, dt):
    """Not a parity bar: the effect of storing the cache in 16 bits, measured
    against the fp32 cache (N(0,1) data, 4096 rows).  bf16 keeps 8 significant
    bits, fp16 11."""
    n_seq, n_pos = 4, 4096
    q = oracle.normal(1400, (n_seq, NH * HD))
    k = oracle.normal(1401, (n_seq, n_pos, KVD))
    v = oracle.normal(1402, (n_seq, n_pos, KVD))
    dq, dout = ctx.upload(q), ctx.empty((n_seq, NH * HD))
    dk, dv = ctx.upload(to16(k, dt)), ctx.upload(to16(v, dt))
    ctx.decode_batched(dq, dk, dv, dout, n_seq, NH, NKV, HD, n_pos, n_pos, kv_dtype=dt)
    offs = np.arange(n_seq, dtype=np.int64) * n_pos
    lens = np.full(n_seq, n_pos, np.int32)
    ref32 = oracle.attention_ragged(q, k.reshape(-1, KVD), v.reshape(-1, KVD), offs, lens, NH, NKV, HD,
                                    n_threads=8)
    err = float(np.abs(dout.numpy() - ref32).max())
    print(f"kv dtype {dt}: max |out16 - out32| = {err:.3e}")
    assert err < (2e-2 if dt == tmac_attn.TMAC_KV_BF16 else 3e-3)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("mfma", [0, 1])
@pytest.mark.parametrize("n_pos,split_len", [(1, 0), (15, 0), (16, 0), (17, 0), (33, 0), (1000, 0), (4096, 0),
                                             (777, 48), (300, 16), (2049, 256)])
def test_decode_mfma_and_valu(ctx, dt, mfma, n_pos, split_len):
    """16-bit decode on the MFMA kernel (default) and on the VALU group kernel:
    partial last tiles, one row, forced short splits (the combine path), and
    rows of very different magnitudes (scores far apart: the lazy max raise)."""
    n_seq = 3
    rng = np.random.default_rng(n_pos + split_len)
    q = oracle.normal(1500 + n_pos, (n_seq, NH * HD))
    k = oracle.normal(1501 + n_pos, (n_seq, n_pos, KVD)) * np.exp2(rng.uniform(-2, 2, (n_seq, n_pos, 1)))
    # small and large query magnitudes (the fp16 path scales q per head); scores stay within ~30 (log2
    # units), where two fp32 evaluations still agree to the contract's 1e-4
    q[0] *= 1e-3
    q[2] *= 4.0
    kb = to16(k.astype(np.float32), dt)
    vb = to16(oracle.normal(1502 + n_pos, (n_seq, n_pos, KVD)), dt)
    dq, dk, dv, dout = ctx.upload(q), ctx.upload(kb), ctx.upload(vb), ctx.empty((n_seq, NH * HD))
    ctx.set_option(tmac_attn.TMAC_OPT_MFMA_DECODE, mfma)
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, tmac_attn.TMAC_KERNEL_GROUP)
    ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, split_len)
    try:
        ctx.decode_batched(dq, dk, dv, dout, n_seq, NH, NKV, HD, n_pos, n_pos, kv_dtype=dt)
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_MFMA_DECODE, 1)
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, 0)
        ctx.set_option(tmac_attn.TMAC_OPT_SPLIT_LEN, 0)
    offs = np.arange(n_seq, dtype=np.int64) * n_pos
    ref = oracle.attention_ragged(q, widen(kb, dt).reshape(-1, KVD), widen(vb, dt).reshape(-1, KVD), offs,
                                  np.full(n_seq, n_pos, np.int32), NH, NKV, HD, n_threads=8)
    assert_close(dout.numpy(), ref, f"dt={dt} mfma={mfma} n_pos={n_pos} split={split_len}")
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("g,kv", [(1, 1), (1, 2), (2, 2), (4, 2), (4, 4), (8, 1)])
def test_decode_mfma_shapes(ctx, dt, g, kv):
    """The MFMA decode at every compiled (query heads per kv head, kv heads)
    shape, batched and ragged, against the oracle on the widened cache."""
    nh, kvd = g * kv, kv * HD
    lens = np.array([700, 1, 33, 2000], np.int32)
    offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
    rows = int(lens.sum())
    q = oracle.normal(1600 + 10 * g + kv, (lens.size, nh * HD))
    kb = to16(oracle.normal(1601 + 10 * g + kv, (rows, kvd)), dt)
    vb = to16(oracle.normal(1602 + 10 * g + kv, (rows, kvd)), dt)
    dq, dk, dv = ctx.upload(q), ctx.upload(kb), ctx.upload(vb)
    doffs, dlens, dout = ctx.upload(offs), ctx.upload(lens), ctx.empty((lens.size, nh * HD))
    ctx.decode_ragged(dq, dk, dv, doffs, dlens, dout, lens.size, nh, kv, HD, int(lens.max()), kv_dtype=dt)
    kw = widen(kb, dt).reshape(-1, kvd)
    vw = widen(vb, dt).reshape(-1, kvd)
    ref = oracle.attention_ragged(q, kw, vw, offs, lens, nh, kv, HD, n_threads=8)
    assert_close(dout.numpy(), ref, f"ragged dt={dt} g={g} kv={kv}")
    n_pos = 1000  # batched: the first 2 * 1000 rows as two sequences
    ctx.decode_batched(dq, dk, dv, dout, 2, nh, kv, HD, n_pos, n_pos, kv_dtype=dt)
    ref = oracle.attention_ragged(q[:2], kw, vw, np.array([0, n_pos], np.int64), np.full(2, n_pos, np.int32), nh,
                                  kv, HD, n_threads=8)
    assert_close(dout.numpy()[:2], ref, f"batched dt={dt} g={g} kv={kv}")
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("dt", [tmac_attn.TMAC_KV_BF16, tmac_attn.TMAC_KV_F16, tmac_attn.TMAC_KV_Q8_0])
@pytest.mark.parametrize("kscale,qscale", [(8.0, 1.0), (1.0, 8.0), (8.0, 0.125), (0.01, 30.0)])
def test_mfma_query_parts_precision(ctx, dt, kscale, qscale):
    """The MFMA decode's query split: three bf16 parts for a bf16 cache (fp32
    exactly), two fp16 parts for fp16 and Q8_0 caches (representation error
    <= 2^-22 |q|).  Keys 8x larger than the query, and the reverse, with
    scores up to a few hundred in log2 units where the lazy max and the exp2
    are most sensitive: still within the fp32 contract on every output."""
    n_seq, n_pos = 4, 2048
    q = oracle.normal(1700, (n_seq, NH * HD)) * np.float32(qscale)
    k = oracle.normal(1701, (n_seq * n_pos, KVD)) * np.float32(kscale)
    v = oracle.normal(1702, (n_seq * n_pos, KVD))
    if dt == tmac_attn.TMAC_KV_Q8_0:
        kb = oracle.q8_kv_rows(k.reshape(-1, HD)).reshape(n_seq * n_pos, -1)
        vb = oracle.q8_kv_rows(v.reshape(-1, HD)).reshape(n_seq * n_pos, -1)
        kw = oracle.q8_kv_widen(kb).reshape(-1, KVD)
        vw = oracle.q8_kv_widen(vb).reshape(-1, KVD)
    else:
        kb, vb = to16(k, dt), to16(v, dt)
        kw, vw = widen(kb, dt).reshape(-1, KVD), widen(vb, dt).reshape(-1, KVD)
    dq, dk, dv, dout = ctx.upload(q), ctx.upload(kb), ctx.upload(vb), ctx.empty((n_seq, NH * HD))
    ctx.decode_batched(dq, dk, dv, dout, n_seq, NH, NKV, HD, n_pos, n_pos, kv_dtype=dt)
    offs = np.arange(n_seq, dtype=np.int64) * n_pos
    ref = oracle.attention_ragged(q, kw, vw, offs, np.full(n_seq, n_pos, np.int32), NH, NKV, HD, n_threads=8)
    assert_close(dout.numpy(), ref, f"dt={dt} keys x{kscale} query x{qscale}")
    assert ctx.check_device_error() == 0
