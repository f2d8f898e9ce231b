"""Pins the oracle's restatement of the reference's quantized projection
(tmac_gguf.cpp:219-231 f16_to_f32, 240-250 dequant_q8_0, 311-327 dequant_q5_0,
510-514 the CPU matmul row loop, 1046-1081 QKV + bias) without running the
reference:

- fp16 decoding against numpy's IEEE conversion over all 65,536 patterns;
- the reference's own Q8_0 GEMV test pattern (test_q8_simdtc.mm:43-56: scale
  1.0, int8 (r*100 + b*10 + l) % 127 - 64, x[i] = i % 7 - 3) at its five shapes
  (test_q8_simdtc.mm:132-136), where every partial sum is an integer below 2^24,
  so the exact answer is an int64 dot product;
- Q5_0 bit placement from single-bit / single-nibble blocks (each element
  reads qh bit e and the low / high nibble of qs[e mod 16]);
- one-hot rows (y = x[j]: catches a transposed or shifted index);
- a float64 evaluation bounding the fp32 row sums on random blocks.
"""
import numpy as np
import pytest

import oracle

F16_ONE = 0x3C00


def q8_block(d_bits: int, q) -> bytes:
    q = np.asarray(q, dtype=np.int8)
    assert q.size == 32
    return bytes([d_bits & 0xFF, d_bits >> 8]) + q.tobytes()


def q5_block(d_bits: int, q5) -> bytes:
    """q5: 32 unsigned 5-bit codes (weight = d * (code - 16))."""
    q5 = np.asarray(q5, dtype=np.int64)
    assert q5.size == 32 and q5.min() >= 0 and q5.max() < 32
    qh = 0
    for e in range(32):
        qh |= int(q5[e] >> 4) << e
    qs = [(int(q5[j]) & 0xF) | ((int(q5[j + 16]) & 0xF) << 4) for j in range(16)]
    return bytes([d_bits & 0xFF, d_bits >> 8]) + qh.to_bytes(4, "little") + bytes(qs)


def reference_q8_pattern(rows: int, cols: int):
    nb = cols // 32
    w = bytearray()
    wi = np.empty((rows, cols), dtype=np.int64)
    for r in range(rows):
        for b in range(nb):
            vals = [(r * 100 + b * 10 + l) % 127 - 64 for l in range(32)]
            wi[r, 32 * b:32 * b + 32] = vals
            w += q8_block(F16_ONE, vals)
    x = np.array([i % 7 - 3 for i in range(cols)], dtype=np.float32)
    return np.frombuffer(bytes(w), dtype=np.uint8), x, wi


def test_f16_to_f32_all_patterns():
    bits = np.arange(65536, dtype=np.uint32)
    want = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    want[0x8000] = 0.0  # the reference's zero branch returns +0 for -0 (tmac_gguf.cpp:224)
    got = np.array([oracle.f16_to_f32(int(h)) for h in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(8, 64), (8, 896), (128, 64), (128, 896), (896, 896)])
def test_q8_0_reference_test_pattern_exact(rows, cols):
    w, x, wi = reference_q8_pattern(rows, cols)
    want = (wi @ x.astype(np.int64)).astype(np.float32)
    got = oracle.matmul_q(oracle.Q8_0, w, x, rows, cols)
    np.testing.assert_array_equal(got, want)


def test_q5_0_bit_placement():
    d = F16_ONE
    zero = q5_block(d, [0] * 32)
    assert [oracle.dequant(oracle.Q5_0, np.frombuffer(zero, np.uint8), e) for e in range(32)] == [-16.0] * 32
    for k in range(32):  # qh bit k lifts element k alone
        blk = bytearray(zero)
        blk[2:6] = (1 << k).to_bytes(4, "little")
        vals = [oracle.dequant(oracle.Q5_0, np.frombuffer(bytes(blk), np.uint8), e) for e in range(32)]
        assert vals == [0.0 if e == k else -16.0 for e in range(32)], k
    for j in range(16):  # low nibble of qs[j] is element j, high nibble element j + 16
        for byte, hit in ((0x0F, j), (0xF0, j + 16)):
            blk = bytearray(zero)
            blk[6 + j] = byte
            vals = [oracle.dequant(oracle.Q5_0, np.frombuffer(bytes(blk), np.uint8), e) for e in range(32)]
            assert vals == [-1.0 if e == hit else -16.0 for e in range(32)], (j, hex(byte))


def test_q5_0_scale_and_codes():
    rng = np.random.default_rng(11)
    for _ in range(20):
        codes = rng.integers(0, 32, 32)
        d16 = np.float16(rng.uniform(-0.05, 0.05))
        blk = np.frombuffer(q5_block(int(d16.view(np.uint16)), codes), np.uint8)
        got = [oracle.dequant(oracle.Q5_0, blk, e) for e in range(32)]
        want = (np.float32(d16) * (codes - 16).astype(np.float32)).tolist()
        assert got == want


@pytest.mark.parametrize("qtype", [oracle.Q5_0, oracle.Q8_0])
def test_one_hot_rows_pick_one_input(qtype):
    rows, cols = 40, 128
    x = np.random.default_rng(3).standard_normal(cols).astype(np.float32)
    w = bytearray()
    for r in range(rows):
        j = (r * 37) % cols
        for b in range(cols // 32):
            if qtype == oracle.Q8_0:
                q = [1 if 32 * b + l == j else 0 for l in range(32)]
                w += q8_block(F16_ONE, q)
            else:
                q = [17 if 32 * b + l == j else 16 for l in range(32)]
                w += q5_block(F16_ONE, q)
    got = oracle.matmul_q(qtype, np.frombuffer(bytes(w), np.uint8), x, rows, cols)
    np.testing.assert_array_equal(got, x[[(r * 37) % cols for r in range(rows)]])


def random_blocks(rng, qtype: int, rows: int, cols: int) -> np.ndarray:
    nb = rows * (cols // 32)
    raw = rng.integers(0, 256, (nb, oracle.BLOCK_BYTES[qtype]), dtype=np.uint8)
    scales = rng.uniform(0.002, 0.05, nb).astype(np.float16) * rng.choice([-1, 1], nb).astype(np.float16)
    raw[:, 0:2] = scales.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


def dequant_f64(qtype: int, w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    nb = cols // 32
    blk = w.reshape(rows, nb, oracle.BLOCK_BYTES[qtype])
    d = blk[:, :, 0:2].copy().view(np.float16).astype(np.float64)  # (rows, nb, 1)
    if qtype == oracle.Q8_0:
        q = blk[:, :, 2:].view(np.int8).astype(np.float64)
    else:
        qh = blk[:, :, 2:6].copy().view(np.uint32).astype(np.int64)  # (rows, nb, 1)
        qs = blk[:, :, 6:22].astype(np.int64)
        lo = np.concatenate([qs & 0xF, qs >> 4], axis=2)
        hi = (qh >> np.arange(32)) & 1
        q = (lo | (hi << 4)).astype(np.float64) - 16
    return (q * d).reshape(rows, cols)


@pytest.mark.parametrize("qtype", [oracle.Q5_0, oracle.Q8_0])
def test_row_sums_against_float64(qtype):
    rng = np.random.default_rng(7 + qtype)
    rows, cols = 96, 896
    w = random_blocks(rng, qtype, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    w64 = dequant_f64(qtype, w, rows, cols)
    y64 = w64 @ x.astype(np.float64)
    got = oracle.matmul_q(qtype, w, x, rows, cols).astype(np.float64)
    # recursive fp32 summation: |error| <= cols * 2^-24 * sum |w x| (+ the rounded products)
    bound = (cols + 1) * 2.0 ** -24 * (np.abs(w64) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(got - y64) <= bound)
    # and the error is that of rounding, not of a wrong term: typical error far below the bound
    assert np.median(np.abs(got - y64) / bound) < 0.05


def test_qkv_adds_present_biases_only():
    rng = np.random.default_rng(5)
    cols, nq, nk, nv = 128, 64, 32, 32
    wq = random_blocks(rng, oracle.Q5_0, nq, cols)
    wk = random_blocks(rng, oracle.Q5_0, nk, cols)
    wv = random_blocks(rng, oracle.Q8_0, nv, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    bq, bv = (rng.standard_normal(n).astype(np.float32) for n in (nq, nv))
    q, k, v = oracle.qkv(wq, wk, wv, True, x, bq, None, bv, nq, nk, nv, cols)
    np.testing.assert_array_equal(q, oracle.matmul_q(oracle.Q5_0, wq, x, nq, cols) + bq)
    np.testing.assert_array_equal(k, oracle.matmul_q(oracle.Q5_0, wk, x, nk, cols))
    np.testing.assert_array_equal(v, oracle.matmul_q(oracle.Q8_0, wv, x, nv, cols) + bv)
    with pytest.raises(ValueError):
        oracle.matmul_q(oracle.Q5_0, wq, x, nq, 100)


# ---- K-quants (tmac_gguf.cpp:330-397), pinned against decoders written from
# GGML's published row dequantisation loops (dequantize_row_q6_K /
# dequantize_row_q4_K: per-128 / per-64-element chunks, get_scale_min_k4),
# whose loop structure differs from the reference's per-element form.

def ggml_q6_k_row(blk: np.ndarray) -> np.ndarray:
    ql, qh = blk[0:128].astype(np.int64), blk[128:192].astype(np.int64)
    sc = blk[192:208].view(np.int8).astype(np.float64)
    d = float(blk[208:210].copy().view(np.float16)[0])
    y = np.empty(256)
    for n in range(2):
        qln, qhn, scn = ql[64 * n:64 * n + 64], qh[32 * n:32 * n + 32], sc[8 * n:8 * n + 8]
        for l in range(32):
            is_ = l // 16
            q1 = ((qln[l] & 0xF) | (((qhn[l] >> 0) & 3) << 4)) - 32
            q2 = ((qln[l + 32] & 0xF) | (((qhn[l] >> 2) & 3) << 4)) - 32
            q3 = ((qln[l] >> 4) | (((qhn[l] >> 4) & 3) << 4)) - 32
            q4 = ((qln[l + 32] >> 4) | (((qhn[l] >> 6) & 3) << 4)) - 32
            y[128 * n + l + 0] = d * scn[is_ + 0] * q1
            y[128 * n + l + 32] = d * scn[is_ + 2] * q2
            y[128 * n + l + 64] = d * scn[is_ + 4] * q3
            y[128 * n + l + 96] = d * scn[is_ + 6] * q4
    return y


def get_scale_min_k4(j: int, q: np.ndarray):
    if j < 4:
        return int(q[j]) & 63, int(q[j + 4]) & 63
    return (int(q[j + 4]) & 0xF) | ((int(q[j - 4]) >> 6) << 4), (int(q[j + 4]) >> 4) | ((int(q[j]) >> 6) << 4)


def ggml_q4_k_row(blk: np.ndarray) -> np.ndarray:
    d = float(blk[0:2].copy().view(np.float16)[0])
    dmin = float(blk[2:4].copy().view(np.float16)[0])
    scales, q = blk[4:16], blk[16:144].astype(np.int64)
    y = np.empty(256)
    is_ = 0
    for j in range(0, 256, 64):
        sc, m = get_scale_min_k4(is_, scales)
        d1, m1 = d * sc, dmin * m
        sc, m = get_scale_min_k4(is_ + 1, scales)
        d2, m2 = d * sc, dmin * m
        qq = q[(j // 64) * 32:(j // 64) * 32 + 32]
        y[j:j + 32] = d1 * (qq & 0xF) - m1
        y[j + 32:j + 64] = d2 * (qq >> 4) - m2
        is_ += 2
    return y


def random_kblocks(rng, qtype: int, n: int) -> np.ndarray:
    raw = rng.integers(0, 256, (n, oracle.BLOCK_BYTES[qtype]), dtype=np.uint8)
    scale = rng.uniform(0.001, 0.02, (n, 2)).astype(np.float16)
    if qtype == oracle.Q6_K:
        raw[:, 208:210] = scale[:, :1].view(np.uint8).reshape(n, 2)
    else:
        raw[:, 0:4] = scale.view(np.uint8).reshape(n, 4)
    return raw


@pytest.mark.parametrize("qtype,ref", [(oracle.Q6_K, ggml_q6_k_row), (oracle.Q4_K, ggml_q4_k_row)])
def test_kquant_dequant_matches_ggml_loops(qtype, ref):
    rng = np.random.default_rng(90 + qtype)
    blocks = random_kblocks(rng, qtype, 12)
    flat = blocks.reshape(-1)
    for b in range(blocks.shape[0]):
        want = ref(blocks[b])
        got = np.array([oracle.dequant(qtype, flat, 256 * b + e) for e in range(256)])
        # every weight is an exact product in fp32 (Q4_K: one rounding of the difference)
        np.testing.assert_allclose(got, want, rtol=2 ** -23, atol=0)


def test_kquant_closed_forms():
    z6 = np.zeros(210, np.uint8)
    z6[208:210] = np.frombuffer(np.float16(1).tobytes(), np.uint8)
    z6[192:208] = 1
    assert [oracle.dequant(oracle.Q6_K, z6, e) for e in range(256)] == [-32.0] * 256
    for e in range(256):  # a single ql nibble lifts one element by 1
        b = z6.copy()
        half, pos = divmod(e, 128)
        sub, l = divmod(pos, 32)
        b[64 * half + l + (32 if sub & 1 else 0)] |= 0x1 if sub < 2 else 0x10
        vals = [oracle.dequant(oracle.Q6_K, b, k) for k in range(256)]
        assert vals == [-31.0 if k == e else -32.0 for k in range(256)], e
    z4 = np.zeros(144, np.uint8)
    z4[0:2] = np.frombuffer(np.float16(1).tobytes(), np.uint8)
    z4[4:8] = 1  # sub-blocks 0-3: scale 1, min 0; 4-7: scale (b[8+j] & 15) = 0
    vals = [oracle.dequant(oracle.Q4_K, z4, e) for e in range(256)]
    assert vals == [0.0] * 256
    z4[16:144] = 0x21  # low nibble 1, high nibble 2
    vals = [oracle.dequant(oracle.Q4_K, z4, e) for e in range(256)]
    assert vals[:128] == [1.0] * 32 + [2.0] * 32 + [1.0] * 32 + [2.0] * 32 and vals[128:] == [0.0] * 128


@pytest.mark.parametrize("qtype", [oracle.Q6_K, oracle.Q4_K])
def test_kquant_matmul_against_float64(qtype):
    rng = np.random.default_rng(95 + qtype)
    rows, cols = 24, 1024
    w = random_kblocks(rng, qtype, rows * cols // 256).reshape(-1)
    x = rng.standard_normal(cols).astype(np.float32)
    ref = ggml_q6_k_row if qtype == oracle.Q6_K else ggml_q4_k_row
    w64 = np.concatenate([ref(b) for b in w.reshape(-1, oracle.BLOCK_BYTES[qtype])]).reshape(rows, cols)
    y64 = w64 @ x.astype(np.float64)
    got = oracle.matmul_q(qtype, w, x, rows, cols).astype(np.float64)
    bound = (cols + 2) * 2.0 ** -24 * (np.abs(w64) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(got - y64) <= bound)
    with pytest.raises(ValueError):
        oracle.matmul_q(qtype, w, x, rows, 896)
