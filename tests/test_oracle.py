"""Pins the CPU oracle (oracle/tmac_oracle.c) -- runs without a GPU.

The reference ships no golden vectors or known-answer tests for this path
(its tests cover only Q8_0 GEMV), so the oracle is pinned by
  * published known-answer vectors for its RNG,
  * closed forms the mathematics fixes (single row, uniform keys, constant
    values, a dominating score, zero query),
  * invariants of GQA attention (group sharing, kv-head isolation, causal
    range, permutation),
  * a float64 brute-force softmax on small shapes, and
  * RoPE identities (pos 0, norm, inverse rotation, pair 0 angle, theta table),
each chosen so that a plausible slip -- a dropped 1/sqrt(d), a wrong kv-head
index, rotate-half instead of adjacent pairs, a sign error -- fails one of them
(the "planted mistake" tests check that explicitly).
"""
import numpy as np
import pytest

import oracle

NH, NKV, HD = 14, 2, 64
G = NH // NKV


def brute_force(q, k, v, n_head, n_kv, hd, past_len, kv_index=None, scale=None):
    """float64 two-pass softmax attention, written independently of the oracle."""
    q = np.asarray(q, np.float64).reshape(n_head, hd)
    k = np.asarray(k, np.float64).reshape(-1, n_kv, hd)[: past_len + 1]
    v = np.asarray(v, np.float64).reshape(-1, n_kv, hd)[: past_len + 1]
    scale = 1.0 / np.sqrt(hd) if scale is None else scale
    out = np.empty((n_head, hd))
    for h in range(n_head):
        kvh = h // (n_head // n_kv) if kv_index is None else kv_index(h)
        s = k[:, kvh, :] @ q[h] * scale
        w = np.exp(s - s.max())
        w /= w.sum()
        out[h] = w @ v[:, kvh, :]
    return out.ravel()


# ------------------------------------------------------------------ RNG
def test_splitmix64_known_answer():
    # Published first outputs of splitmix64 seeded with 1234567.
    assert oracle.splitmix64(1234567, 5) == [
        6457827717110365317, 3203168211198807973, 9817491932198370423,
        4593380528125082431, 16408922859458223821]


def test_xoshiro256starstar_known_answer():
    # Published first outputs of xoshiro256** from state {1, 2, 3, 4}.
    assert oracle.xoshiro256ss([1, 2, 3, 4], 10) == [
        11520, 0, 1509978240, 1215971899390074240, 1216172134540287360, 607988272756665600,
        16172922978634559625, 8476171486693032832, 10595114339597558777, 2904607092377533576]


def test_normal_stream_statistics_and_determinism():
    x = oracle.normal(1, 400_000)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.var()) - 1.0) < 0.01
    assert abs(float(((x - x.mean()) ** 3).mean())) < 0.02
    np.testing.assert_array_equal(x[:1000], oracle.normal(1, 1000))
    assert not np.array_equal(oracle.normal(2, 1000), x[:1000])


# ------------------------------------------------------------------ attention closed forms
def test_single_row_returns_v_exactly():
    q = oracle.normal(3, NH * HD)
    k = oracle.normal(4, (1, NKV * HD))
    v = oracle.normal(5, (1, NKV * HD))
    out = oracle.attention(q, k, v, NH, NKV, HD, 0).reshape(NH, HD)
    for h in range(NH):
        np.testing.assert_array_equal(out[h], v[0].reshape(NKV, HD)[h // G])


def test_equal_keys_give_mean_of_values():
    n = 37
    q = oracle.normal(6, NH * HD)
    k = np.tile(oracle.normal(7, (1, NKV * HD)), (n, 1))
    v = oracle.normal(8, (n, NKV * HD))
    out = oracle.attention(q, k, v, NH, NKV, HD, n - 1).reshape(NH, HD)
    mean = v.astype(np.float64).reshape(n, NKV, HD).mean(axis=0)
    for h in range(NH):
        np.testing.assert_allclose(out[h], mean[h // G], rtol=0, atol=2e-6)


def test_constant_values_are_returned():
    n = 100
    q = oracle.normal(9, NH * HD)
    k = oracle.normal(10, (n, NKV * HD))
    u = oracle.normal(11, NKV * HD)
    v = np.tile(u, (n, 1))
    out = oracle.attention(q, k, v, NH, NKV, HD, n - 1).reshape(NH, HD)
    for h in range(NH):
        np.testing.assert_allclose(out[h], u.reshape(NKV, HD)[h // G], rtol=2e-6, atol=1e-7)


def test_dominating_score_selects_its_row_exactly():
    n, hot = 50, 23
    q = np.zeros(NH * HD, np.float32)
    q[::HD] = 1.0  # every head looks at dim 0 only
    k = np.zeros((n, NKV * HD), np.float32)
    k[hot, ::HD] = 8.0 * 130.0  # score 130 (after /sqrt(64)) vs 0 elsewhere: exp(-130) underflows
    v = oracle.normal(12, (n, NKV * HD))
    out = oracle.attention(q, k, v, NH, NKV, HD, n - 1).reshape(NH, HD)
    for h in range(NH):
        np.testing.assert_array_equal(out[h], v[hot].reshape(NKV, HD)[h // G])


def test_zero_query_is_uniform_average():
    n = 64
    k = oracle.normal(13, (n, NKV * HD))
    v = oracle.normal(14, (n, NKV * HD))
    out = oracle.attention(np.zeros(NH * HD, np.float32), k, v, NH, NKV, HD, n - 1).reshape(NH, HD)
    mean = v.astype(np.float64).reshape(n, NKV, HD).mean(axis=0)
    for h in range(NH):
        np.testing.assert_allclose(out[h], mean[h // G], atol=2e-6)


# ------------------------------------------------------------------ attention invariants
def test_equal_queries_in_a_group_give_equal_outputs():
    n = 40
    q = oracle.normal(15, (NH, HD))
    q[1] = q[0]
    q[9] = q[8]
    k = oracle.normal(16, (n, NKV * HD))
    v = oracle.normal(17, (n, NKV * HD))
    out = oracle.attention(q, k, v, NH, NKV, HD, n - 1).reshape(NH, HD)
    np.testing.assert_array_equal(out[0], out[1])
    np.testing.assert_array_equal(out[8], out[9])
    assert not np.array_equal(out[0], out[8])


def test_kv_head_isolation():
    """Heads 0..6 read only kv head 0 (tmac_gguf.cpp:1099 kv = qh / 7)."""
    n = 30
    q = oracle.normal(18, NH * HD)
    k = oracle.normal(19, (n, NKV, HD))
    v = oracle.normal(20, (n, NKV, HD))
    a = oracle.attention(q, k, v, NH, NKV, HD, n - 1).reshape(NH, HD)
    k2, v2 = k.copy(), v.copy()
    k2[:, 1] += 3.0
    v2[:, 1] *= -2.0
    b = oracle.attention(q, k2, v2, NH, NKV, HD, n - 1).reshape(NH, HD)
    np.testing.assert_array_equal(a[:G], b[:G])
    assert np.abs(a[G:] - b[G:]).max() > 0.1


def test_rows_after_past_len_are_ignored():
    n, cap = 20, 32
    q = oracle.normal(21, NH * HD)
    k = oracle.normal(22, (cap, NKV * HD))
    v = oracle.normal(23, (cap, NKV * HD))
    a = oracle.attention(q, k[:n], v[:n], NH, NKV, HD, n - 1)
    k[n:] = np.nan
    v[n:] = np.nan
    b = oracle.attention(q, k, v, NH, NKV, HD, n - 1)
    np.testing.assert_array_equal(a, b)


def test_row_permutation_changes_only_rounding():
    n = 77
    q = oracle.normal(24, NH * HD)
    k = oracle.normal(25, (n, NKV * HD))
    v = oracle.normal(26, (n, NKV * HD))
    perm = np.random.default_rng(0).permutation(n)
    a = oracle.attention(q, k, v, NH, NKV, HD, n - 1)
    b = oracle.attention(q, k[perm], v[perm], NH, NKV, HD, n - 1)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------ brute force
@pytest.mark.parametrize("n_head,n_kv,n", [(14, 2, 1), (14, 2, 9), (14, 2, 64), (4, 4, 33), (8, 1, 17), (6, 2, 50)])
def test_oracle_matches_float64_brute_force(n_head, n_kv, n):
    q = oracle.normal(100 + n, n_head * HD)
    k = oracle.normal(200 + n, (n, n_kv * HD))
    v = oracle.normal(300 + n, (n, n_kv * HD))
    got = oracle.attention(q, k, v, n_head, n_kv, HD, n - 1)
    ref = brute_force(q, k, v, n_head, n_kv, HD, n - 1)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)


def test_planted_mistakes_are_detected():
    """The brute-force check distinguishes the plausible slips it is meant to catch."""
    n = 48
    q = oracle.normal(31, NH * HD)
    k = oracle.normal(32, (n, NKV * HD))
    v = oracle.normal(33, (n, NKV * HD))
    got = oracle.attention(q, k, v, NH, NKV, HD, n - 1)
    wrong_kv = brute_force(q, k, v, NH, NKV, HD, n - 1, kv_index=lambda h: h % NKV)
    no_scale = brute_force(q, k, v, NH, NKV, HD, n - 1, scale=1.0)
    for bad in (wrong_kv, no_scale):
        assert np.abs(got - bad).max() > 1e-2


# ------------------------------------------------------------------ RoPE
def test_rope_pos0_is_identity():
    x = oracle.normal(40, NH * HD)
    np.testing.assert_array_equal(oracle.rope_heads(x, NH, HD, 0), x)


def test_rope_theta_table():
    t = oracle.rope_theta(HD, 1e6).astype(np.float64)
    ref = 1e6 ** (-np.arange(0, HD, 2) / HD)
    assert t[0] == 1.0
    np.testing.assert_allclose(t, ref, rtol=3e-7)


@pytest.mark.parametrize("pos", [1, 17, 255, 4095])
def test_rope_preserves_pair_norms_and_inverts(pos):
    x = oracle.normal(41 + pos, NKV * HD)
    y = oracle.rope_heads(x, NKV, HD, pos)
    n0 = np.hypot(x[0::2].astype(np.float64), x[1::2])
    n1 = np.hypot(y[0::2].astype(np.float64), y[1::2])
    np.testing.assert_allclose(n1, n0, rtol=1e-6)
    back = oracle.rope_heads(y, NKV, HD, -pos)
    np.testing.assert_allclose(back, x, rtol=1e-5, atol=2e-6)


def test_rope_adjacent_pairs_and_pair0_angle():
    """GPT-J adjacent pairs (d, d+1), not rotate-half; pair 0 turns by exactly pos radians."""
    pos = 3
    x = np.zeros(HD, np.float32)
    x[0] = 1.0
    y = oracle.rope_heads(x, 1, HD, pos)
    np.testing.assert_allclose(y[:2], [np.cos(pos), np.sin(pos)], rtol=1e-6)
    assert np.all(y[2:] == 0)  # rotate-half would put sin() at dim 32
    x = np.zeros(HD, np.float32)
    x[2] = 1.0  # pair 1: theta = 1e6^(-2/64)
    y = oracle.rope_heads(x, 1, HD, pos)
    th = pos * 1e6 ** (-2 / 64)
    np.testing.assert_allclose(y[2:4], [np.cos(th), np.sin(th)], rtol=2e-6)


# ------------------------------------------------------------------ cache write / layer step / drivers
def test_cache_write_touches_one_row_bytewise():
    cache = np.full((8, NKV * HD), 7.25, np.float32)
    src = oracle.normal(50, NKV * HD)
    oracle.cache_write(cache, 5, src)
    np.testing.assert_array_equal(cache[5], src)
    assert np.all(cache[np.arange(8) != 5] == 7.25)


def test_layer_step_is_rope_then_write_then_attention():
    cap, pos = 16, 11
    kc = oracle.normal(51, (cap, NKV * HD))
    vc = oracle.normal(52, (cap, NKV * HD))
    q = oracle.normal(53, NH * HD)
    kn = oracle.normal(54, NKV * HD)
    vn = oracle.normal(55, NKV * HD)
    k1, v1 = kc.copy(), vc.copy()
    out, rq, rk = oracle.layer_step(q, kn, vn, k1, v1, NH, NKV, HD, pos)
    q2, k2 = oracle.rope(q, kn, NH, NKV, HD, pos)
    np.testing.assert_array_equal(rq, q2)
    np.testing.assert_array_equal(rk, k2)
    kc[pos], vc[pos] = k2, vn
    np.testing.assert_array_equal(k1, kc)
    np.testing.assert_array_equal(v1, vc)
    np.testing.assert_array_equal(out, oracle.attention(q2, kc, vc, NH, NKV, HD, pos))


def test_decode_step_equals_layer_steps_in_turn():
    """The whole-step driver (the reference's per-layer loop) equals one
    layer_step per layer, each on its own cache slice, bit for bit; the timing
    build gives the same result within the fp32 bar."""
    L, cap, pos = 3, 20, 13
    kc = oracle.normal(61, (L, cap, NKV * HD))
    vc = oracle.normal(62, (L, cap, NKV * HD))
    q = oracle.normal(63, (L, NH * HD))
    kn = oracle.normal(64, (L, NKV * HD))
    vn = oracle.normal(65, (L, NKV * HD))
    k1, v1 = kc.copy(), vc.copy()
    out = oracle.decode_step(q, kn, vn, k1, v1, NH, NKV, HD, pos)
    for layer in range(L):
        k2, v2 = kc[layer].copy(), vc[layer].copy()
        ref, _, _ = oracle.layer_step(q[layer], kn[layer], vn[layer], k2, v2, NH, NKV, HD, pos)
        np.testing.assert_array_equal(out[layer], ref)
        np.testing.assert_array_equal(k1[layer], k2)
        np.testing.assert_array_equal(v1[layer], v2)
    k3, v3 = kc.copy(), vc.copy()
    out_t = oracle.decode_step(q, kn, vn, k3, v3, NH, NKV, HD, pos, timing=True)
    assert np.all(np.abs(out_t - out) <= 2e-5 + 1e-4 * np.abs(out))
    with pytest.raises(ValueError):
        oracle.decode_step(q, kn, vn, kc.copy(), vc.copy(), NH, NKV, HD, cap)


def test_ragged_driver_equals_single_sequence_calls():
    lens = np.array([1, 5, 40, 3], np.int32)
    offs = np.array([0, 1, 6, 46], np.int64)
    k = oracle.normal(56, (49, NKV * HD))
    v = oracle.normal(57, (49, NKV * HD))
    q = oracle.normal(58, (4, NH * HD))
    got = oracle.attention_ragged(q, k, v, offs, lens, NH, NKV, HD, n_threads=4)
    for s in range(4):
        o, n = offs[s], lens[s]
        np.testing.assert_array_equal(got[s], oracle.attention(q[s], k[o:o + n], v[o:o + n], NH, NKV, HD, n - 1))


def test_prefill_rows_are_decode_at_prefix_plus_i():
    n_seq, n_q, prefix, cap = 2, 5, 7, 16
    k = oracle.normal(60, (n_seq, cap, NKV * HD))
    v = oracle.normal(61, (n_seq, cap, NKV * HD))
    q = oracle.normal(62, (n_seq, n_q, NH * HD))
    got = oracle.prefill(q, k, v, n_seq, n_q, prefix, cap, NH, NKV, HD, n_threads=2)
    for s in range(n_seq):
        for i in range(n_q):
            np.testing.assert_array_equal(got[s, i], oracle.attention(q[s, i], k[s], v[s], NH, NKV, HD, prefix + i))


def test_bad_arguments_are_rejected():
    q = np.zeros(NH * HD, np.float32)
    k = np.zeros((4, NKV * HD), np.float32)
    with pytest.raises(ValueError):
        oracle.attention(q, k, k, NH, 3, HD, 2)
    with pytest.raises(ValueError):
        oracle.attention(q, k, k, NH, NKV, HD, -1)


def test_build_flags_match_makefile():
    """oracle.BUILD_FLAGS (reported with the CPU baseline) are the flags oracle/Makefile compiles with."""
    import os
    import re
    mk = open(os.path.join(os.path.dirname(oracle.__file__), "Makefile")).read()
    lines = [" ".join(l.replace("\\\n", " ").split()) for l in re.findall(r"\$\(CC\)[^\n]*(?:\\\n[^\n]*)*", mk)]
    for name, flags in oracle.BUILD_FLAGS.items():
        words = flags.split()[1:]
        assert any(all(w in ln.split() for w in words) for ln in lines), (name, flags, lines)
