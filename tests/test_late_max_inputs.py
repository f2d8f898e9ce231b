"""CPU checks of the late-rising-max inputs (tests/late_max.py) used by
tests/test_gpu_late_max.py.

They show, in float64 and on the fp32 inputs the GPU tests upload, that:
  * each planted row beats every row before it by the planted height, for every
    query head, so any pass over the rows in order (a wave's steps, a split, a
    stream-K segment, a prefill tile pair) must raise its running max there by
    more than the 8-log2-unit threshold of the kernels' lazy rescale;
  * a row planted 160 log2 units up makes the oracle (tmac_gguf.cpp:1093-1128)
    return that row's V exactly, the closed form the GPU tests hold the kernels to;
  * a model of the lazy online softmax (raise the max only when a score beats it by
    more than 8, rescaling the sums) matches the oracle on these inputs, while the
    same model without the rescale -- the defect of kernel_flash_attn.metal:76-79 --
    fails on them and passes on plain N(0, 1) inputs, so these inputs, unlike
    N(0, 1) ones, detect a missing or wrong rescale.
"""
import numpy as np
import pytest

import late_max as lm
import oracle
from conftest import assert_close

NH, NKV, HD = 14, 2, 64
TAU = 8.0


def lazy_softmax(q, k, v, n_head, n_kv, hd, order, rescale=True):
    """Online softmax over rows in `order`, base 2, the max raised only when a score beats it
    by more than TAU (all heads of the pass share one decision, as a wave does).  Returns
    (out [n_head][hd], number of raises after the first row)."""
    s = lm.scores_log2(q, k, n_head, n_kv, hd)
    g = n_head // n_kv
    vv = np.asarray(v, np.float64).reshape(-1, n_kv, hd)
    m = np.full(n_head, -np.inf)
    l = np.zeros(n_head)
    acc = np.zeros((n_head, hd))
    late = 0
    for i, p in enumerate(order):
        sp = s[:, p]
        if np.any(sp - m > TAU):
            mn = np.maximum(m, sp)
            if rescale:
                alpha = np.where(np.isinf(m), 0.0, np.exp2(m - mn))
                l *= alpha
                acc *= alpha[:, None]
            m = mn
            late += i > 0
        e = np.exp2(sp - m)
        l += e
        for h in range(n_head):
            acc[h] += e[h] * vv[p, h // g]
    return (acc / l[:, None]).astype(np.float32), late


def c1_like(seed, n=256):
    q = oracle.normal(seed, NH * HD)
    k = oracle.normal(seed + 1, (n, NKV * HD))
    v = oracle.normal(seed + 2, (n, NKV * HD))
    return q, k, v


def test_planted_rows_rise_by_their_height():
    q, k, v = c1_like(8100)
    rows = [40, 100, 180, 255]
    kp = lm.plant(q, k, rows, [9, 18, 27, 36], NH, NKV, HD)
    margins = lm.rise_margins(q, kp, rows, NH, NKV, HD)
    assert np.all(margins > 8.9) and np.all(margins < 9.1), margins
    # rows not planted are unchanged
    other = np.setdiff1d(np.arange(k.shape[0]), rows)
    np.testing.assert_array_equal(kp[other], k[other])


def test_planted_rows_survive_q8_storage():
    """The staircase and the dominating row of the paged tests, after Q8_0 storage
    (int8 per element, one fp16 scale per 32): each planted row still beats every row
    before it by more than 8.5 log2 units, and the dominating row every other row by
    more than 150, on the widened rows the kernels and the oracle read."""
    q = oracle.normal(8700, (2, NH * HD))
    k0 = lm.plant(q[0], oracle.normal(8710, (4096, NKV * HD)), [15, 16, 1023, 1024, 4095], [9, 18, 27, 36, 45],
                  NH, NKV, HD)
    k1 = lm.plant(q[1], oracle.normal(8711, (3000, NKV * HD)), [2048], [160], NH, NKV, HD)
    w0 = oracle.q8_kv_widen(oracle.q8_kv_rows(k0.reshape(-1, HD))).reshape(k0.shape)
    w1 = oracle.q8_kv_widen(oracle.q8_kv_rows(k1.reshape(-1, HD))).reshape(k1.shape)
    assert np.all(lm.rise_margins(q[0], w0, [15, 16, 1023, 1024, 4095], NH, NKV, HD) > 8.5)
    assert lm.dominance(q[1], w1, 2048, NH, NKV, HD) > 150


@pytest.mark.parametrize("row", [0, 77, 255])
def test_dominating_row_gives_its_v_exactly(row):
    q, k, v = c1_like(8200)
    kp = lm.plant(q, k, [row], [160], NH, NKV, HD)
    assert lm.dominance(q, kp, row, NH, NKV, HD) > 150
    out = oracle.attention(q, kp, v, NH, NKV, HD, k.shape[0] - 1).reshape(NH, HD)
    for h in range(NH):
        kv = h // (NH // NKV)
        np.testing.assert_array_equal(out[h], v[row, kv * HD:(kv + 1) * HD])


def test_common_direction_plant_rises_for_every_query():
    """Prefill planting: queries q + 4, key rows lambda * ones with lambda 1, 1.6, 2.4, 3.5:
    each planted row beats every earlier row by more than 9 log2 units for every query
    row and head that sees it."""
    n_q, cap = 64, 300
    q = lm.common_queries(oracle.normal(8300, (n_q, NH * HD)), 4.0)
    k = oracle.normal(8301, (cap, NKV * HD))
    rows = [100, 150, 236, 299]
    kp = lm.plant_common(k, rows, [1.0, 1.6, 2.4, 3.5])
    for i in range(n_q):
        m = lm.rise_margins(q[i], kp, rows, NH, NKV, HD)
        assert np.all(m > 9), (i, m)


def test_lazy_model_detects_missing_rescale_only_on_planted_inputs():
    q, k, v = c1_like(8400)
    order = np.arange(k.shape[0])
    ref = oracle.attention(q, k, v, NH, NKV, HD, k.shape[0] - 1).reshape(NH, HD)
    good, late = lazy_softmax(q, k, v, NH, NKV, HD, order)
    bad, _ = lazy_softmax(q, k, v, NH, NKV, HD, order, rescale=False)
    assert late == 0  # N(0, 1): no raise after the first row ...
    assert_close(good, ref, "lazy model, N(0,1)")
    assert_close(bad, ref, "no-rescale model, N(0,1)")  # ... so a missing rescale goes unseen

    for rows, levels in (([255], [9]), ([128], [9]), ([60, 130, 200, 255], [9, 18, 27, 36])):
        kp = lm.plant(q, k, rows, levels, NH, NKV, HD)
        ref = oracle.attention(q, kp, v, NH, NKV, HD, k.shape[0] - 1).reshape(NH, HD)
        for stride in (1, 4, 8):  # a sequential pass, and the rows of one wave of 4 or 8
            for w in range(stride):
                sub = order[w::stride]
                good, late = lazy_softmax(q, kp[sub], v[sub], NH, NKV, HD, np.arange(sub.size))
                if any(r in sub for r in rows):
                    assert late >= 1, (rows, stride, w)
        good, _ = lazy_softmax(q, kp, v, NH, NKV, HD, order)
        bad, _ = lazy_softmax(q, kp, v, NH, NKV, HD, order, rescale=False)
        assert_close(good, ref, f"lazy model, rows {rows}")
        with pytest.raises(AssertionError):
            assert_close(bad, ref, f"no-rescale model, rows {rows}")


def test_gain_ramp_raises_late():
    q, k, v = c1_like(8500, n=4096)
    kp = lm.gain_ramp(k, 3.0)
    _, late = lazy_softmax(q, kp, v, NH, NKV, HD, np.arange(4096))
    assert late >= 1
    q30 = (q * 30).astype(np.float32)
    _, late = lazy_softmax(q30, k, v, NH, NKV, HD, np.arange(4096))
    assert late >= 1
