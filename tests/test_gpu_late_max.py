"""GPU parity on inputs whose online-softmax running max rises late.

Every kernel keeps a lazy running max: it is raised, and the running sums
rescaled, only when a score beats it by more than kTau = 8 log2 units (a
wave-uniform branch).  With q, k ~ N(0, 1) no score does so after the first
step, so plain inputs never run that branch late.  The inputs here do
(tests/late_max.py; their effect is checked in float64 on the CPU by
tests/test_late_max_inputs.py):
  * staircase: key rows planted 9, 18, 27, ... log2 units above every other row
    for every query head, on ascending rows: the wave, split or segment that
    holds each such row must raise its max there by 9 > 8 and rescale what it
    has summed so far (weights up to 2^-9 of the new max, so a missing or wrong
    rescale moves the output far outside the tolerance);
  * one row 9 above the rest at the last row (or at a split / segment / tile
    pair boundary): the raise happens on the last step, with the rows before it
    still carrying a large share of the weight;
  * a dominating row, 160 log2 (111 natural) units above the rest: its weight is
    1 and every other weight underflows to 0, so the output must equal that row's
    V exactly, the closed form of tmac_gguf.cpp:1114-1126 (expf(s - L), L = s_max);
  * keys scaled up along the sequence (gain 1 -> 3) and queries scaled by 30:
    maxima that keep rising to the end, drawn at random.
Branches reached (tmac_gguf.cpp_amd/csrc/attn_kernels.hip): attend() `over >
kTau` (the group kernel: C3 headline launch, C4 unit grid, stream-K; the head
kernel), hv_body `sc - m > kTau` (split-V head kernel: attention_op at C1, the
C2 layer step), any_body `mx - m > kTau` (any-shape kernel), prefill_body
`(tm - m) * c > kTau` (C5), mdecode_segment's back() `tm - m > kTau` (MFMA
decode of bf16 / fp16 / Q8_0 caches); the same branches over paged caches
(pages scattered in random pool order, planted rows on page boundaries) in the
paged decode and the batched paged layer step.  The reference's own GPU kernel fails on
exactly this class of input (kernel_flash_attn.metal:76-79).

Oracle: oracle/tmac_oracle.c (tmac_gguf.cpp:990-1016, 1090-1091, 1093-1128).
Tolerance: |gpu - ref| <= 2e-5 + 1e-4 |ref|; dominating rows bit-exact.
"""
import numpy as np
import pytest

import late_max as lm
import oracle
import tmac_attn
import workloads
from conftest import assert_close
from test_gpu_kv_q8_paged import PR, build_pool, store, widen

pytestmark = pytest.mark.gpu
NH, NKV, HD = 14, 2, 64
G = NH // NKV
QD, KVD = NH * HD, NKV * HD


def bf16_round(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


def assert_v_row(out_seq, v_row, what, n_head=NH, n_kv=NKV, hd=HD):
    """Every query head's output equals its kv head's half of v_row, bit for bit."""
    out_seq = np.asarray(out_seq, np.float32).reshape(n_head, hd)
    g = n_head // n_kv
    for h in range(n_head):
        kv = h // g
        np.testing.assert_array_equal(out_seq[h].view(np.uint32), np.asarray(v_row[kv * hd:(kv + 1) * hd],
                                      np.float32).view(np.uint32), err_msg=f"{what}: head {h}")


# Plans: name -> function(q_seq, k_seq) returning (k_seq', q_seq', dominating row or None).
def plans_for(n):
    return {
        "last+9": lambda q, k: (lm.plant(q, k, [n - 1], [9], NH, NKV, HD), q, None),
        "mid+9": lambda q, k: (lm.plant(q, k, [n // 2 - 1], [9], NH, NKV, HD), q, None),
        "stairs": lambda q, k: (lm.plant(q, k, [n // 4 - 6, n // 2 + 1, 3 * n // 4 + 2, n - 1], [9, 18, 27, 36],
                                         NH, NKV, HD), q, None),
        "stairs-last-step": lambda q, k: (lm.plant(q, k, [n - 4, n - 3, n - 2, n - 1], [9, 18, 27, 36], NH, NKV,
                                                   HD), q, None),
        "dom-last": lambda q, k: (lm.plant(q, k, [n - 1], [160], NH, NKV, HD), q, n - 1),
        "dom-mid": lambda q, k: (lm.plant(q, k, [n // 2 + 2], [160], NH, NKV, HD), q, n // 2 + 2),
        "gain3": lambda q, k: (lm.gain_ramp(k, 3.0), q, None),
        "q30": lambda q, k: (k, (q * 30).astype(np.float32), None),
    }


@pytest.fixture(scope="module")
def c3_late():
    """Config 3 inputs with sequences 0..7 carrying the eight plans (the rest N(0, 1))."""
    n_seq, n_pos = 256, 4096
    q, k, v = workloads.c3(n_seq, n_pos)
    dom = {}
    for s, (name, f) in enumerate(plans_for(n_pos).items()):
        rows = slice(s * n_pos, (s + 1) * n_pos)
        k[rows], q[s], d = f(q[s], k[rows])
        if d is not None:
            dom[s] = d
    return q, k, v, dom


def test_config3_headline_launch_late_max(ctx, c3_late):
    """The config-3 headline launch (256 x 4096, one split per sequence: the 4-wave
    group kernel, whose waves take every 4th 4-row step) with sequences 0..7
    carrying late raises: at the last row, in the middle, a four-step staircase
    spread over different waves, four raises inside the last step, dominating
    rows at the last and a middle row (exact V), a gain ramp and q x 30.  All 256
    sequences against the oracle."""
    q, k, v, dom = c3_late
    n_seq, n_pos = 256, 4096
    info, n_cu = ctx.device_info()
    if n_cu == 256:
        assert ctx.query_split(n_seq, n_pos, NH, NKV) == (4096, 1)
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    dout = ctx.empty((n_seq, QD))
    dout.fill_bytes(0xFF)
    ctx.decode_batched(dq, dk, dv, dout, n_seq, NH, NKV, HD, n_pos, n_pos)
    got = dout.numpy()
    for d in (dq, dk, dv, dout):
        d.free()
    offs = np.arange(n_seq, dtype=np.int64) * n_pos
    ref = oracle.attention_ragged(q, k, v, offs, np.full(n_seq, n_pos, np.int32), NH, NKV, HD, n_threads=16)
    names = list(plans_for(n_pos))
    for s in range(len(names)):
        assert_close(got[s], ref[s], f"config 3 sequence {s} ({names[s]})")
    assert_close(got, ref, "config 3, all sequences")
    for s, r in dom.items():
        assert_v_row(got[s], v[s * n_pos + r], f"config 3 sequence {s} dominating row {r}")
        assert_v_row(ref[s], v[s * n_pos + r], f"oracle, sequence {s}")
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("dt", ["bf16", "f16", "q8"])
def test_config3_narrow_caches_late_max(ctx, c3_late, dt):
    """The same 256 x 4096 inputs on bf16 / fp16 / Q8_0 caches: the MFMA decode,
    whose waves take every 4th (8th for Q8_0) 16-row tile and raise a column's max
    when one of its lanes' 4 keys beats it by more than 8.  Oracle on the widened
    cache; dominating rows give the widened V row exactly."""
    q, k, v, dom = c3_late
    n_seq, n_pos = 256, 4096
    if dt == "q8":
        code = tmac_attn.TMAC_KV_Q8_0
        kb = oracle.q8_kv_rows(k.reshape(-1, HD)).reshape(-1, NKV * oracle.Q8_HEAD_BYTES)
        vb = oracle.q8_kv_rows(v.reshape(-1, HD)).reshape(-1, NKV * oracle.Q8_HEAD_BYTES)
        kw = oracle.q8_kv_widen(kb).reshape(-1, KVD)
        vw = oracle.q8_kv_widen(vb).reshape(-1, KVD)
    elif dt == "f16":
        code = tmac_attn.TMAC_KV_F16
        kb, vb = k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
        kw, vw = kb.view(np.float16).astype(np.float32), vb.view(np.float16).astype(np.float32)
    else:
        code = tmac_attn.TMAC_KV_BF16
        kw, vw = bf16_round(k), bf16_round(v)
        kb, vb = (kw.view(np.uint32) >> 16).astype(np.uint16), (vw.view(np.uint32) >> 16).astype(np.uint16)
    dq, dk, dv = ctx.upload(q), ctx.upload(kb), ctx.upload(vb)
    dout = ctx.empty((n_seq, QD))
    dout.fill_bytes(0xFF)
    ctx.decode_batched(dq, dk, dv, dout, n_seq, NH, NKV, HD, n_pos, n_pos, kv_dtype=code)
    got = dout.numpy()
    for d in (dq, dk, dv, dout):
        d.free()
    offs = np.arange(n_seq, dtype=np.int64) * n_pos
    ref = oracle.attention_ragged(q, kw, vw, offs, np.full(n_seq, n_pos, np.int32), NH, NKV, HD, n_threads=16)
    names = list(plans_for(n_pos))
    for s in range(len(names)):
        assert_close(got[s], ref[s], f"{dt} cache, sequence {s} ({names[s]})")
    assert_close(got, ref, f"{dt} cache, all sequences")
    for s, r in dom.items():
        assert lm.dominance(q[s], kw[s * n_pos:(s + 1) * n_pos], r, NH, NKV, HD) > 150
        assert_v_row(got[s], vw[s * n_pos + r], f"{dt} cache, sequence {s} dominating row {r}")
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("kernel", [tmac_attn.TMAC_KERNEL_AUTO, tmac_attn.TMAC_KERNEL_HEAD,
                                    tmac_attn.TMAC_KERNEL_GROUP])
@pytest.mark.parametrize("plan", list(plans_for(256)))
def test_config1_attention_op_late_max(ctx, kernel, plan):
    """Config 1 (attention_op, 256 rows, query at 255) with each plan: the automatic
    kernel is the split-V head kernel (8 waves, 8-row steps of one kv head, every
    8th step per wave), also forced onto the head kernel and the group kernel."""
    q, k, v = workloads.c1()
    k, q, dom = plans_for(256)[plan](q, k)
    ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, kernel)
    try:
        dq, dk, dv, dout = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.empty(QD)
        ctx.attention_op(dq, dk, dv, dout, NH, NKV, HD, 255)
        got = dout.numpy()
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_KERNEL, tmac_attn.TMAC_KERNEL_AUTO)
    ref = oracle.attention(q, k, v, NH, NKV, HD, 255)
    assert_close(got, ref, f"config 1 {plan} kernel {kernel}")
    if dom is not None:
        assert_v_row(got, v[dom], f"config 1 {plan} kernel {kernel}")
    for d in (dq, dk, dv, dout):
        d.free()
    assert ctx.check_device_error() == 0


# Config 2: steps (positions) at which layers 0 and 3 get a new token planted
# above every cached row (9 log2 units; 160 at DOM_STEP, whose output is v_new).
C2_RAISE_STEPS = (1, 9, 64, 127, 128, 200, 254, 255)
C2_DOM_STEP = 150


def test_config2_graph_late_max(ctx):
    """The captured config-2 step (fused layer launches + position advance, the
    split-V head kernel in layer mode) replayed for every position 0..255 of four
    layers.  In layers 0 and 3 the new token of several steps is planted 9 log2
    units above every cached row (160 at one step): the token is attended last,
    from registers, so the raise happens on a wave's final step, and the planted
    rows then stay in the cache as high-norm keys that later queries meet at
    random.  Every output against the oracle; the dominating step's output equals
    v_new exactly; both caches bit-exact at the end."""
    L, cap = 4, 256
    q, kn, vn = workloads.c2(L, cap)
    kc = ctx.upload(np.zeros((L, cap, KVD), np.float32))
    vc = ctx.upload(np.zeros((L, cap, KVD), np.float32))
    ref_k = np.zeros((L, cap, KVD), np.float32)
    ref_v = np.zeros((L, cap, KVD), np.float32)
    dq, dkn, dvn, dout = ctx.empty((L, QD)), ctx.empty((L, KVD)), ctx.empty((L, KVD)), ctx.empty((L, QD))
    pos = ctx.upload(np.zeros(1, np.int32))
    ctx.rope_prepare(HD, 1e6, cap)
    s = ctx.stream()
    ctx.step_begin(s)
    for i in range(L):
        ctx.layer_attention_devpos(dq.at(i * QD), dkn.at(i * KVD), dvn.at(i * KVD), kc.at(i * cap * KVD),
                                   vc.at(i * cap * KVD), dout.at(i * QD), NH, NKV, HD, pos, cap, 1e6, stream=s)
    ctx.pos_update(pos, 1, add=True, stream=s)
    g = ctx.step_end(s)
    try:
        for step in range(cap):
            for i in (0, 3):
                if step in C2_RAISE_STEPS or step == C2_DOM_STEP:
                    level = 160.0 if step == C2_DOM_STEP else 9.0
                    q_rot = oracle.rope_heads(q[step, i], NH, HD, step, 1e6)
                    base = lm.scores_log2(q_rot, ref_k[i, :step], NH, NKV, HD).max(axis=1)
                    qh = q[step, i].reshape(NH, HD)
                    for kv in range(NKV):
                        hs = slice(kv * G, (kv + 1) * G)
                        kn[step, i, kv * HD:(kv + 1) * HD] = lm.key_for_scores(
                            qh[hs], kn[step, i, kv * HD:(kv + 1) * HD], base[hs] + level, HD).astype(np.float32)
            dq.copy_from(q[step])
            dkn.copy_from(kn[step])
            dvn.copy_from(vn[step])
            ctx.graph_launch(g, s)
            ctx.synchronize(s)
            got = dout.numpy()
            for i in range(L):
                ref, _, _ = oracle.layer_step(q[step, i], kn[step, i], vn[step, i], ref_k[i], ref_v[i], NH, NKV, HD,
                                              step, 1e6)
                assert_close(got[i], ref, f"config 2 step {step} layer {i}")
                if step == C2_DOM_STEP and i in (0, 3):
                    assert_v_row(got[i], vn[step, i], f"config 2 dominating step {step} layer {i}")
                    assert_v_row(ref, vn[step, i], "oracle")
        np.testing.assert_array_equal(kc.numpy(), ref_k)
        np.testing.assert_array_equal(vc.numpy(), ref_v)
    finally:
        ctx.graph_destroy(g)
        ctx.destroy_stream(s)
        for d in (kc, vc, dq, dkn, dvn, dout, pos):
            d.free()
    assert ctx.check_device_error() == 0


def _c4_unit_len(n_cu, lens):
    """Split length of the unit-grid ragged decode with the total_rows hint (the host's
    choose_split: 4-wave workgroups, rows per split = ceil(total / (CUs - n_seq)) rounded up
    to a 16-row round)."""
    per = -(-int(lens.sum()) // (n_cu - lens.size))
    return -(-per // 16) * 16


def _c4_sk_bounds(n_cu, lens):
    """Stream-K range starts inside each sequence: (sequence, row) pairs where a workgroup's
    range [u S, (u + 1) S) of the 16-row padded row space begins."""
    padded = -(-lens.astype(np.int64) // 16) * 16
    R = int(padded.sum())
    per = -(-R // n_cu)
    S = max(-(-per // 16) * 16, 64)
    first = np.concatenate([[0], np.cumsum(padded)[:-1]])
    out = []
    for u in range(1, n_cu):
        b = u * S
        s = int(np.searchsorted(first, b, side="right") - 1)
        if 0 < b - first[s] < lens[s]:
            out.append((s, int(b - first[s])))
    return out


def test_config4_late_max_all_schedules(ctx):
    """Config 4 (16 ragged sequences, 255,714 rows) with late raises placed on the
    split boundaries of each schedule: the unit grid with the total_rows hint
    (splits of 1,072 rows on 256 CUs), without it (2,048 rows), and stream-K
    (equal ranges of the padded row space, one workgroup per CU).  Dominating rows
    sit on the first row of a split, on the last row of one and on a stream-K
    range start (their sequences' outputs equal those V rows exactly in every
    schedule, which needs the cross-split merge to drop every other split), and
    staircases climb across split boundaries."""
    q, k, v, offs, lens = workloads.c4()
    info, n_cu = ctx.device_info()
    S1, S2 = _c4_unit_len(n_cu, lens), 2048
    sk = _c4_sk_bounds(n_cu, lens)
    order = np.argsort(-lens)  # longest first
    plans = {}
    a, b, c, d, e, f = (int(x) for x in order[:6])
    plans[a] = ([S1 - 1, S1, 2 * S2 - 1, 2 * S2, int(lens[a]) - 1], [9, 18, 27, 36, 45])
    plans[b] = ([2 * S1], [160])
    plans[c] = ([S2 - 1], [160])
    plans[d] = ([int(lens[d]) - 1], [9])
    sk_in = [(s, r) for s, r in sk if s not in plans]
    if sk_in:
        s0, r0 = sk_in[0]
        plans[s0] = ([r0], [160])
    for s, (rows, levels) in plans.items():
        assert max(rows) < lens[s], (s, rows, int(lens[s]))
        seg = slice(int(offs[s]), int(offs[s]) + int(lens[s]))
        k[seg] = lm.plant(q[s], k[seg], rows, levels, NH, NKV, HD)
    k[int(offs[e]):int(offs[e]) + int(lens[e])] = lm.gain_ramp(k[int(offs[e]):int(offs[e]) + int(lens[e])], 3.0)
    q[f] = q[f] * 30
    dom = {s: rows[0] for s, (rows, levels) in plans.items() if levels[0] >= 150}
    total = int(lens.sum())
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    doff, dlen = ctx.upload(offs), ctx.upload(lens)
    dout = ctx.empty((lens.size, QD))
    ref = oracle.attention_ragged(q, k, v, offs, lens, NH, NKV, HD, n_threads=16)
    try:
        for name, hint, stream_k in (("unit grid, hint", total, 0), ("unit grid, no hint", 0, 0),
                                     ("stream-K", 0, 2), ("default", total, 1)):
            ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, stream_k)
            dout.fill_bytes(0xFF)
            ctx.decode_ragged(dq, dk, dv, doff, dlen, dout, lens.size, NH, NKV, HD, 32768, total_rows=hint)
            got = dout.numpy()
            assert_close(got, ref, f"config 4 late max, {name}")
            for s, r in dom.items():
                assert_v_row(got[s], v[int(offs[s]) + r], f"config 4 {name}: sequence {s} dominating row {r}")
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 1)
        for x in (dq, dk, dv, doff, dlen, dout):
            x.free()
    assert ctx.check_device_error() == 0


ANY_SHAPES = [(14, 2, 128), (3, 1, 64), (9, 3, 66), (14, 2, 32)]


@pytest.mark.parametrize("nh,nkv,hd", ANY_SHAPES)
def test_any_shape_late_max(ctx, nh, nkv, hd):
    """The any-shape kernel (8 waves, 2-row steps, each wave every 8th step) through
    attention_op over 1001 rows and the fused layer step at position 1000: a
    staircase ending on the last row, a dominating middle row (exact V), and a new
    token planted 9 (then 160: exact v_new) above every cached row."""
    n = 1001
    g = nh // nkv
    q = oracle.normal(8600 + hd, nh * hd)
    k = oracle.normal(8601 + hd, (n, nkv * hd))
    v = oracle.normal(8602 + hd, (n, nkv * hd))
    dq, dv, dout = ctx.upload(q), ctx.upload(v), ctx.empty(nh * hd)
    for rows, levels in (([100, 499, 777, 1000], [9, 18, 27, 36]), ([640], [160]), ([1000], [9])):
        kp = lm.plant(q, k, rows, levels, nh, nkv, hd)
        dk = ctx.upload(kp)
        ctx.attention_op(dq, dk, dv, dout, nh, nkv, hd, n - 1)
        got = dout.numpy()
        assert_close(got, oracle.attention(q, kp, v, nh, nkv, hd, n - 1), f"any shape {nh}/{nkv}/{hd} rows {rows}")
        if levels[0] >= 150:
            assert_v_row(got, v[rows[0]], f"any shape {nh}/{nkv}/{hd}", nh, nkv, hd)
        dk.free()
    # the fused layer step at position 1000: the new token attended last
    cap, pos = 1024, 1000
    ctx.rope_prepare(hd, 1e6, cap)
    for level in (9.0, 160.0):
        kc = np.zeros((cap, nkv * hd), np.float32)
        vc = np.zeros((cap, nkv * hd), np.float32)
        kc[:pos], vc[:pos] = k[:pos], v[:pos]
        kn = oracle.normal(8610 + hd, nkv * hd)
        vn = oracle.normal(8611 + hd, nkv * hd)
        q_rot = oracle.rope_heads(q, nh, hd, pos, 1e6)
        base = lm.scores_log2(q_rot, kc[:pos], nh, nkv, hd).max(axis=1)
        qh = q.reshape(nh, hd)
        for kv in range(nkv):
            hs = slice(kv * g, (kv + 1) * g)
            kn[kv * hd:(kv + 1) * hd] = lm.key_for_scores(qh[hs], kn[kv * hd:(kv + 1) * hd], base[hs] + level,
                                                          hd).astype(np.float32)
        dkc, dvc, dkn, dvn = ctx.upload(kc), ctx.upload(vc), ctx.upload(kn), ctx.upload(vn)
        ctx.layer_attention(dq, dkn, dvn, dkc, dvc, dout, nh, nkv, hd, pos, cap, 1e6)
        got = dout.numpy()
        ref, _, _ = oracle.layer_step(q, kn, vn, kc, vc, nh, nkv, hd, pos, 1e6)
        assert_close(got, ref, f"any shape layer step {nh}/{nkv}/{hd} new token +{level}")
        np.testing.assert_array_equal(dkc.numpy(), kc)
        if level >= 150:
            assert_v_row(got, vn, f"any shape layer step {nh}/{nkv}/{hd}", nh, nkv, hd)
        for x in (dkc, dvc, dkn, dvn):
            x.free()
    for x in (dq, dv, dout):
        x.free()
    assert ctx.check_device_error() == 0


def test_config5_prefill_late_max_all_rows(ctx):
    """Config 5 (4 x 512 queries after a 1536-row prefix) with every query given a
    common component (q + 4) and planted key rows lambda * ones, which score
    lambda * sum(q) / 8 for every query and head that sees them:
      sequence 0: a staircase on the last prefix row, the first query's own row, both
        sides of a 128-key tile pair boundary, a middle row and the last row -- each
        9+ log2 units above every earlier row for every query row that sees it (checked
        in float64 below), so the kernel's wave raises its max on late tile pairs,
        including the causal-diagonal pair;
      sequence 1: a dominating row (key 1700): every query at or past it returns
        bf16(V[1700]) to within 2^-21 relative (the oracle returns it exactly; the
        kernel's weight of the top key is exp2(s c - round(m c)), whose argument is
        the rounding residual of m c rather than 0, so it is 1 +- 1e-5, split into
        bf16 hi + lo, and divided out again by the row sum of the same parts);
      sequence 2: keys scaled up along the sequence (x1 -> x3), plain queries;
      sequence 3: plain keys, queries x 30.
    All 4 x 512 rows against the oracle on the bf16-rounded inputs."""
    n_seq, n_q, prefix = 4, 512, 1536
    cap = prefix + n_q
    q, k, v = workloads.c5(n_seq, n_q, prefix)
    stairs = [1535, 1536, 1663, 1664, 1800, 2047]
    lambdas = [1.2, 1.8, 2.6, 3.6, 4.9, 6.6]
    q[0] = lm.common_queries(q[0], 4.0)
    k[0] = lm.plant_common(k[0], stairs, lambdas)
    q[1] = lm.common_queries(q[1], 4.0)
    k[1] = lm.plant_common(k[1], [1700], [6.0])
    k[2] = lm.gain_ramp(k[2], 3.0)
    q[3] = q[3] * 30
    qb, kb, vb = bf16_round(q), bf16_round(k), bf16_round(v)
    # the planted rows rise as stated, for every query row that sees them
    for i in range(0, n_q, 7):
        seen = [r for r in stairs if r <= prefix + i]
        m = lm.rise_margins(qb[0, i], kb[0], seen, NH, NKV, HD)
        assert np.all(m > 9), (i, m)
        if prefix + i >= 1700:
            assert lm.dominance(qb[1, i], kb[1, :prefix + i + 1], 1700, NH, NKV, HD) > 150
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    dout = ctx.empty((n_seq, n_q, QD))
    ctx.prefill(dq, dk, dv, dout, n_seq, n_q, prefix, cap, NH, NKV, HD)
    got = dout.numpy()
    for d in (dq, dk, dv, dout):
        d.free()
    ref = oracle.prefill(qb, kb, vb, n_seq, n_q, prefix, cap, NH, NKV, HD, n_threads=16)
    for s in range(n_seq):
        assert_close(got[s], ref[s], f"config 5 late max, sequence {s}")
    want = np.repeat(vb[1, 1700].reshape(1, NKV, 1, HD), G, axis=2).reshape(QD)
    for i in range(1700 - prefix, n_q):
        np.testing.assert_array_equal(ref[1, i], want)
        err = np.abs(got[1, i].astype(np.float64) - want)
        assert np.all(err <= 2.0 ** -21 * np.abs(want)), (i, float((err / np.abs(want)).max()))
    assert ctx.check_device_error() == 0


PAGED_DT = {"f32": tmac_attn.TMAC_KV_F32, "q8": tmac_attn.TMAC_KV_Q8_0}


@pytest.mark.parametrize("dt", ["f32", "q8"])
@pytest.mark.parametrize("stream_k", [0, 2])
def test_paged_decode_late_max(ctx, dt, stream_k):
    """Paged decode over 16-row pages scattered in random pool order -- the group
    kernel (fp32 cache) and the MFMA kernel (Q8_0 cache), on the unit grid and on
    stream-K -- with staircases across page boundaries (rows 15 | 16, 1023 | 1024)
    up to the last row, a dominating row on a page boundary (row 2048; exact V), a
    dominating last row, a raise at the last row, q x 30 and a gain ramp.  Oracle on
    the rows gathered through the block table and widened to fp32."""
    code = PAGED_DT[dt]
    lens = np.array([4096, 3000, 1537, 700, 64, 17], np.int32)
    n_seq = lens.size
    q = oracle.normal(8700, (n_seq, QD))
    rows = [oracle.normal(8710 + s, (int(lens[s]), KVD)) for s in range(n_seq)]
    vrows = [oracle.normal(8730 + s, (int(lens[s]), KVD)) for s in range(n_seq)]
    rows[0] = lm.plant(q[0], rows[0], [15, 16, 1023, 1024, 4095], [9, 18, 27, 36, 45], NH, NKV, HD)
    rows[1] = lm.plant(q[1], rows[1], [2048], [160], NH, NKV, HD)
    rows[2] = lm.plant(q[2], rows[2], [1536], [9], NH, NKV, HD)
    rows[3] = lm.plant(q[3], rows[3], [699], [160], NH, NKV, HD)
    q[4] = q[4] * 30
    rows[5] = lm.gain_ramp(rows[5], 3.0)
    k_st = [store(r, code) for r in rows]
    v_st = [store(r, code) for r in vrows]
    n_pages = int(sum((l + PR - 1) // PR for l in lens)) + 7
    kp, table = build_pool(k_st, code, n_pages, np.random.default_rng(87))
    vp, _ = build_pool(v_st, code, n_pages, np.random.default_rng(87))
    kw = [widen(r, code) for r in k_st]
    vw = [widen(r, code) for r in v_st]
    assert lm.dominance(q[1], kw[1], 2048, NH, NKV, HD) > 150
    assert lm.dominance(q[3], kw[3], 699, NH, NKV, HD) > 150
    dq, dk, dv, dtab, dl = ctx.upload(q), ctx.upload(kp), ctx.upload(vp), ctx.upload(table), ctx.upload(lens)
    dout = ctx.empty((n_seq, QD))
    ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, stream_k)
    try:
        ctx.decode_paged(dq, dk, dv, n_pages, dtab, table.shape[1], dl, dout, n_seq, NH, NKV, HD, int(lens.max()),
                         total_rows=int(lens.sum()), kv_dtype=code)
        got = dout.numpy()
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 1)
    offs = np.concatenate([[0], np.cumsum(lens[:-1])]).astype(np.int64)
    ref = oracle.attention_ragged(q, np.concatenate(kw), np.concatenate(vw), offs, lens, NH, NKV, HD, n_threads=8)
    assert_close(got, ref, f"paged {dt} stream_k={stream_k}")
    assert_v_row(got[1], vw[1][2048], f"paged {dt}: dominating row 2048")
    assert_v_row(got[3], vw[3][699], f"paged {dt}: dominating last row")
    for d in (dq, dk, dv, dtab, dl, dout):
        d.free()
    assert ctx.check_device_error() == 0


@pytest.mark.parametrize("dt", ["f32", "q8"])
@pytest.mark.parametrize("stream_k", [0, 2])
def test_paged_layer_step_late_max(ctx, dt, stream_k):
    """The batched paged layer step (RoPE, the new row written into its page,
    attention over rows 0..pos): the new token of some sequences is planted 9 (and,
    for one, 160) log2 units above every cached row, so the segment or split that
    takes the new token raises its max on its last row; positions at and around
    page boundaries.  Unit grid and stream-K (fp32); Q8_0 on the MFMA kernel."""
    code = PAGED_DT[dt]
    positions = np.array([16, 1023, 2047, 300, 15, 999], np.int32)
    levels = [9.0, 9.0, 160.0, 9.0, 9.0, None]
    n_seq = positions.size
    max_len = int(positions.max()) + 1
    k_st = [store(oracle.normal(8800 + s, (int(p) + 1, KVD)), code) for s, p in enumerate(positions)]
    v_st = [store(oracle.normal(8820 + s, (int(p) + 1, KVD)), code) for s, p in enumerate(positions)]
    n_pages = int(sum((p + PR) // PR for p in positions)) + 5
    kp, table = build_pool(k_st, code, n_pages, np.random.default_rng(88))
    vp, _ = build_pool(v_st, code, n_pages, np.random.default_rng(88))
    q = oracle.normal(8840, (n_seq, QD))
    kn = oracle.normal(8841, (n_seq, KVD))
    vn = oracle.normal(8842, (n_seq, KVD))
    for s, (p, lev) in enumerate(zip(positions, levels)):
        if lev is None:
            continue
        rows = np.array([table[s, r // PR] * PR + r % PR for r in range(int(p))])
        q_rot = oracle.rope_heads(q[s], NH, HD, int(p), 1e6)
        base = lm.scores_log2(q_rot, widen(kp[rows], code), NH, NKV, HD).max(axis=1)
        qh = q[s].reshape(NH, HD)
        for kv in range(NKV):
            hs = slice(kv * G, (kv + 1) * G)
            kn[s, kv * HD:(kv + 1) * HD] = lm.key_for_scores(qh[hs], kn[s, kv * HD:(kv + 1) * HD],
                                                              base[hs] + lev, HD).astype(np.float32)
    dq, dkn, dvn = ctx.upload(q), ctx.upload(kn), ctx.upload(vn)
    dk, dv, dtab, dpos = ctx.upload(kp), ctx.upload(vp), ctx.upload(table), ctx.upload(positions)
    dout = ctx.empty((n_seq, QD))
    ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, stream_k)
    try:
        ctx.layer_attention_paged(dq, dkn, dvn, dk, dv, n_pages, dtab, table.shape[1], dpos, dout, n_seq, NH, NKV,
                                  HD, max_len, 1e6, kv_dtype=code)
        got, kp_got = dout.numpy(), dk.numpy()
    finally:
        ctx.set_option(tmac_attn.TMAC_OPT_STREAM_K, 1)
    kp_ref, vp_ref = kp.copy(), vp.copy()
    for s, p in enumerate(positions):
        qr, kr = oracle.rope(q[s], kn[s], NH, NKV, HD, int(p), 1e6)
        row = table[s, p // PR] * PR + p % PR
        kp_ref[row] = store(kr, code)[0]
        vp_ref[row] = store(vn[s], code)[0]
        rows = np.array([table[s, r // PR] * PR + r % PR for r in range(int(p) + 1)])
        ref = oracle.attention(qr, widen(kp_ref[rows], code), widen(vp_ref[rows], code), NH, NKV, HD, int(p))
        assert_close(got[s], ref, f"paged layer {dt} stream_k={stream_k} seq {s} pos {p}")
        if levels[s] is not None and levels[s] >= 150:
            assert_v_row(got[s], widen(vp_ref[row:row + 1], code)[0], f"paged layer {dt}: dominating new token")
    np.testing.assert_array_equal(kp_got, kp_ref)
    for d in (dq, dkn, dvn, dk, dv, dtab, dpos, dout):
        d.free()
    assert ctx.check_device_error() == 0
