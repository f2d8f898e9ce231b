"""Pins the oracle's restatement of the reference's Q8_0 requantizer, the
format of the Q8_0 KV cache (scripts/extract_tmac.py:53-74 float_to_fp16,
159-173 quantize_q8_0_block), without running the reference:

- float_to_fp16 known answers: exact fp16 values keep their bits, the
  mantissa is truncated (one value where IEEE rounding differs), fp16
  subnormals flush to a signed zero, exponents >= 2^16 give infinity;
- truncation against numpy's float16 conversion stepped toward zero, over
  random normal-range values (a different mechanism, same answer);
- block known answers with d = 1 exactly (max |x| = 127): q = x rounded half
  to even (0.5 -> 0, 1.5 -> 2, 2.5 -> 2, -63.5 -> -64), all-zero and tiny
  blocks (max |x| < 1e-10 -> d = 1, q = 0);
- invariants on random blocks of every scale: the max element maps to +-127,
  |x / d - q| <= 1/2, q keeps the sign of x, scale bits = float_to_fp16(d);
- the KV head-row layout against the reference block stream read back with
  dequant_q8_0 (tmac_gguf.cpp:240-250, pinned in test_oracle_quant.py).
"""
import numpy as np
import pytest

import oracle


def test_f16_trunc_known_answers():
    for v, bits in [(1.0, 0x3C00), (-2.0, 0xC000), (65504.0, 0x7BFF), (0.5, 0x3800), (2.0 ** -14, 0x0400),
                    (0.333251953125, 0x3555)]:
        assert oracle.f32_to_f16_trunc(v) == bits, v
    assert oracle.f32_to_f16_trunc(1.0 + 3 * 2.0 ** -12) == 0x3C00  # IEEE nearest gives 0x3C01
    assert np.float16(1.0 + 3 * 2.0 ** -12).view(np.uint16) == 0x3C01
    assert oracle.f32_to_f16_trunc(65535.0) == 0x7BFF       # exponent 0x8E: truncated, not rounded to inf
    assert oracle.f32_to_f16_trunc(65536.0) == 0x7C00       # exponent 0x8F: infinity
    assert oracle.f32_to_f16_trunc(-1e6) == 0xFC00
    assert oracle.f32_to_f16_trunc(2.0 ** -15) == 0         # fp16 subnormal range: flushed
    assert oracle.f32_to_f16_trunc(-2.0 ** -15) == 0x8000   # ... keeping the sign
    assert oracle.f32_to_f16_trunc(0.0) == 0 and oracle.f32_to_f16_trunc(-0.0) == 0
    assert oracle.f32_to_f16_trunc(1e-45) == 0              # fp32 subnormal


def test_f16_trunc_is_numpy_rounded_toward_zero():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(4000) * np.exp2(rng.uniform(-13, 15, 4000))).astype(np.float32)
    x = x[(np.abs(x) >= 2.0 ** -14) & (np.abs(x) < 65504)]  # fp16's normal range (the rest is pinned above)
    assert x.size > 3000
    for v in x:
        h = np.float16(v)
        if abs(float(h)) > abs(float(v)):  # numpy rounded away from zero: step back one ulp
            h = (h.view(np.uint16) - 1).astype(np.uint16).view(np.float16)
        assert oracle.f32_to_f16_trunc(v) == int(h.view(np.uint16)), v


def test_q8_block_known_answers():
    x = np.zeros(32, np.float32)
    x[:6] = [127, -63.5, 0.5, 1.5, 2.5, -0.5]
    b = oracle.quantize_q8_0_block(x)
    assert b[0] == 0x00 and b[1] == 0x3C  # d = 1.0
    assert list(b[2:8].view(np.int8)) == [127, -64, 0, 2, 2, 0]
    assert not b[8:].any()
    zero = oracle.quantize_q8_0_block(np.zeros(32, np.float32))
    assert list(zero[:2]) == [0x00, 0x3C] and not zero[2:].any()
    tiny = np.full(32, 1e-11, np.float32)
    assert list(oracle.quantize_q8_0_block(tiny)) == [0x00, 0x3C] + [0] * 32
    # max |x| = 1e-10 is not "< 1e-10" (float32(1e-10) lies above 1e-10): d = 1e-10 / 127, far
    # below fp16's normal range, so the stored scale is 0 while q still spans +-127.
    edge = np.zeros(32, np.float32)
    edge[3], edge[4] = np.float32(1e-10), -np.float32(5e-11)
    be = oracle.quantize_q8_0_block(edge)
    assert be[0] == 0 and be[1] == 0 and be[2 + 3].view(np.int8) == 127 and be[2 + 4].view(np.int8) in (-64, -63)


@pytest.mark.parametrize("scale", [1e-3, 0.05, 1.0, 37.0, 3000.0])
def test_q8_block_invariants(scale):
    rng = np.random.default_rng(int(scale * 1000) + 5)
    for _ in range(200):
        x = (rng.standard_normal(32) * scale).astype(np.float32)
        b = oracle.quantize_q8_0_block(x)
        q = b[2:].view(np.int8).astype(np.int64)
        amax = float(np.abs(x).max())
        d = np.float32(np.float32(amax) / np.float32(127.0))
        assert int(b[0]) | (int(b[1]) << 8) == oracle.f32_to_f16_trunc(d)
        i = int(np.abs(x).argmax())
        assert q[i] == (127 if x[i] > 0 else -127)
        assert np.all(np.abs(q) <= 127)
        assert np.all((q == 0) | (np.sign(q) == np.sign(x)))
        assert np.all(np.abs(x.astype(np.float64) / float(d) - q) <= 0.5 + 1e-6)


def test_q8_kv_rows_layout_and_widen():
    rng = np.random.default_rng(21)
    n = 37
    x = (rng.standard_normal((n, 64)) * np.exp2(rng.uniform(-4, 4, (n, 1)))).astype(np.float32)
    rows = oracle.q8_kv_rows(x)
    assert rows.shape == (n, oracle.Q8_HEAD_BYTES)
    stream = np.concatenate([oracle.quantize_q8_0_block(x[r, 32 * b:32 * b + 32]) for r in range(n) for b in (0, 1)])
    blocks = stream.reshape(n, 2, 34)
    np.testing.assert_array_equal(rows[:, :32], blocks[:, 0, 2:])
    np.testing.assert_array_equal(rows[:, 32:64], blocks[:, 1, 2:])
    np.testing.assert_array_equal(rows[:, 64:66], blocks[:, 0, :2])
    np.testing.assert_array_equal(rows[:, 66:68], blocks[:, 1, :2])
    wide = oracle.q8_kv_widen(rows)
    ref = np.array([oracle.dequant(oracle.Q8_0, stream, e) for e in range(n * 64)], np.float32)
    np.testing.assert_array_equal(wide, ref)
    # round trip: within half a step of the stored scale plus the truncation of the scale
    d_true = np.abs(x.reshape(n, 2, 32)).max(axis=2) / 127.0
    d_st = np.array([[oracle.f16_to_f32(int(rows[r, 64 + 2 * b]) | (int(rows[r, 65 + 2 * b]) << 8))
                      for b in (0, 1)] for r in range(n)])
    err = np.abs(wide.reshape(n, 2, 32) - x.reshape(n, 2, 32)).max(axis=2)
    assert np.all(err <= 0.5 * d_st + 127.0 * (d_true - d_st) + 1e-6 * d_true)
