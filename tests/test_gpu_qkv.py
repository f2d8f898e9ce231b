"""GPU parity of the QKV projection (tmac_fused_qkv_op / tmac_fused_qkv_bias),
the output projection (tmac_matmul_q5_0 / _q8_0 / tmac_matmul_add) and
elem_op op 0 against the oracle (tmac_gguf.cpp:1046-1081, 510-514, 1497-1499).

Bars:
- integer-valued weights and inputs (the reference's own Q8_0 test pattern,
  test_q8_simdtc.mm:43-56, and a Q5_0 analogue) make every partial sum an exact
  integer, so the GPU result must equal the oracle bit for bit whatever the
  summation order;
- real-valued weights at the magnitudes of a Q5_0 Qwen2-0.5B checkpoint
  (|d| <= 0.004) use the fp32 tolerance |gpu - ref| <= 2e-5 + 1e-4 |ref|;
- large-magnitude weights use the summation bound of two fp32 sums in different
  orders: |gpu - ref| <= 2 * (cols + 1) * 2^-24 * sum_j |w_j x_j|.
"""
import numpy as np
import pytest

import oracle
import tmac_attn
from conftest import assert_close
from test_oracle_quant import dequant_f64, q5_block, random_blocks, reference_q8_pattern

pytestmark = pytest.mark.gpu
F16_ONE = 0x3C00


def q5_integer_pattern(rows: int, cols: int, salt: int = 0):
    nb = cols // 32
    w = bytearray()
    wi = np.empty((rows, cols), dtype=np.int64)
    for r in range(rows):
        for b in range(nb):
            codes = [(r * 7 + b * 5 + 3 * l + salt) % 32 for l in range(32)]
            wi[r, 32 * b:32 * b + 32] = np.array(codes) - 16
            w += q5_block(F16_ONE, codes)
    return np.frombuffer(bytes(w), dtype=np.uint8), wi


def run_qkv(ctx, wq, wk, wv, x, nq, nk, nv, cols, v_is_q8, bias=(None, None, None), with_bias=None):
    dw = [ctx.upload(w) if w is not None and w.size else None for w in (wq, wk, wv)]
    dx = ctx.upload(x)
    dy = [ctx.empty(max(n, 1)) for n in (nq, nk, nv)]
    db = [None if b is None else ctx.upload(b) for b in bias]
    ctx.fused_qkv(dw[0], dw[1], dw[2], dx, dy[0], dy[1], dy[2], nq, nk, nv, cols, v_is_q8,
                  b_q=db[0], b_k=db[1], b_v=db[2], with_bias=with_bias)
    out = [d.numpy()[:n] for d, n in zip(dy, (nq, nk, nv))]
    for d in dw + [dx] + dy + db:
        if d is not None:
            d.free()
    return out


@pytest.mark.parametrize("rows,cols", [(8, 64), (8, 896), (128, 64), (128, 896), (896, 896)])
def test_q8_0_reference_pattern_bit_exact(ctx, rows, cols):
    """The reference's Q8_0 GEMV test (scale 1, integer weights and inputs) on the V segment."""
    w, x, wi = reference_q8_pattern(rows, cols)
    _, _, got = run_qkv(ctx, None, None, w, x, 0, 0, rows, cols, True)
    np.testing.assert_array_equal(got, oracle.matmul_q(oracle.Q8_0, w, x, rows, cols))
    np.testing.assert_array_equal(got, (wi @ x.astype(np.int64)).astype(np.float32))


@pytest.mark.parametrize("rows,cols", [(8, 64), (37, 896), (128, 2048), (5, 32)])
def test_q5_0_integer_pattern_bit_exact(ctx, rows, cols):
    wq, wiq = q5_integer_pattern(rows, cols)
    wk, wik = q5_integer_pattern(3, cols, salt=1)
    wv, wiv = q5_integer_pattern(2, cols, salt=2)
    x = np.array([i % 7 - 3 for i in range(cols)], dtype=np.float32)
    q, k, v = run_qkv(ctx, wq, wk, wv, x, rows, 3, 2, cols, False)
    for got, wi, name in ((q, wiq, "q"), (k, wik, "k"), (v, wiv, "v")):
        np.testing.assert_array_equal(got, (wi @ x.astype(np.int64)).astype(np.float32), err_msg=name)


def qwen_like(rng, qtype, rows, cols):
    w = random_blocks(rng, qtype, rows, cols)
    nb = rows * (cols // 32)
    blk = w.reshape(nb, oracle.BLOCK_BYTES[qtype])
    d = (rng.uniform(0.0005, 0.004, nb) * rng.choice([-1, 1], nb)).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    return blk.reshape(-1)


@pytest.mark.parametrize("v_is_q8", [True, False])
def test_qwen2_shape_with_bias_matches_oracle(ctx, v_is_q8):
    """One layer at the Qwen2-0.5B shape: 896 q rows, 128 k, 128 v, 896 inputs, biases."""
    rng = np.random.default_rng(21 + v_is_q8)
    cols, nq, nk, nv = 896, 896, 128, 128
    wq = qwen_like(rng, oracle.Q5_0, nq, cols)
    wk = qwen_like(rng, oracle.Q5_0, nk, cols)
    wv = qwen_like(rng, oracle.Q8_0 if v_is_q8 else oracle.Q5_0, nv, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    bias = tuple(rng.standard_normal(n).astype(np.float32) * 0.1 for n in (nq, nk, nv))
    got = run_qkv(ctx, wq, wk, wv, x, nq, nk, nv, cols, v_is_q8, bias)
    ref = oracle.qkv(wq, wk, wv, v_is_q8, x, *bias, nq, nk, nv, cols)
    for g, r, name in zip(got, ref, "qkv"):
        assert_close(g, r, f"{name} (v_is_q8={v_is_q8})")
    # without bias: the other entry point
    got0 = run_qkv(ctx, wq, wk, wv, x, nq, nk, nv, cols, v_is_q8)
    ref0 = oracle.qkv(wq, wk, wv, v_is_q8, x, None, None, None, nq, nk, nv, cols)
    for g, r, name in zip(got0, ref0, "qkv"):
        assert_close(g, r, f"{name} no bias (v_is_q8={v_is_q8})")


@pytest.mark.parametrize("qtype", [oracle.Q5_0, oracle.Q8_0])
def test_large_magnitude_within_summation_bound(ctx, qtype):
    rng = np.random.default_rng(31 + qtype)
    rows, cols = 77, 1536
    w = random_blocks(rng, qtype, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    _, _, got = run_qkv(ctx, None, None, w, x, 0, 0, rows, cols, qtype == oracle.Q8_0)
    ref = oracle.matmul_q(qtype, w, x, rows, cols)
    scale = np.abs(dequant_f64(qtype, w, rows, cols)) @ np.abs(x.astype(np.float64))
    bound = 2 * (cols + 1) * 2.0 ** -24 * scale
    assert np.all(np.abs(got.astype(np.float64) - ref) <= bound)


def test_partial_biases_and_ragged_row_counts(ctx):
    """Row totals that do not fill the last workgroup, a missing k bias."""
    rng = np.random.default_rng(41)
    cols, nq, nk, nv = 96, 13, 5, 3
    wq, wk = qwen_like(rng, oracle.Q5_0, nq, cols), qwen_like(rng, oracle.Q5_0, nk, cols)
    wv = qwen_like(rng, oracle.Q8_0, nv, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    bq, bv = rng.standard_normal(nq).astype(np.float32), rng.standard_normal(nv).astype(np.float32)
    got = run_qkv(ctx, wq, wk, wv, x, nq, nk, nv, cols, True, (bq, None, bv))
    ref = oracle.qkv(wq, wk, wv, True, x, bq, None, bv, nq, nk, nv, cols)
    for g, r, name in zip(got, ref, "qkv"):
        assert_close(g, r, name)


def test_rejects_bad_arguments(ctx):
    d = ctx.empty(1024)
    qkv = lambda **kw: ctx.fused_qkv(*(kw.get(n, d) for n in ("wq", "wk", "wv", "x", "yq", "yk", "yv")),
                                      kw.get("nq", 4), kw.get("nk", 4), kw.get("nv", 4), kw.get("cols", 64),
                                      True, check=False)
    assert qkv(cols=48) == tmac_attn.TMAC_ERR_INVALID_ARG
    assert qkv(cols=0) == tmac_attn.TMAC_ERR_INVALID_ARG
    assert qkv(nq=-1) == tmac_attn.TMAC_ERR_INVALID_ARG
    assert qkv(wk=None) == tmac_attn.TMAC_ERR_NULL_POINTER
    assert qkv(x=d.at(1)) == tmac_attn.TMAC_ERR_MISALIGNED
    assert qkv(nq=0, nk=0, nv=0) == tmac_attn.TMAC_OK


def test_elem_op_add_bit_exact(ctx):
    rng = np.random.default_rng(51)
    a = rng.standard_normal(1000).astype(np.float32)
    b = rng.standard_normal(1000).astype(np.float32)
    da, db = ctx.upload(a), ctx.upload(b)
    ctx.elem_op(0, da, db, 1000)
    np.testing.assert_array_equal(da.numpy(), a + b)
    assert ctx.elem_op(1, da, db, 1000, check=False) == tmac_attn.TMAC_ERR_UNSUPPORTED


@pytest.mark.parametrize("qtype", [oracle.Q5_0, oracle.Q8_0])
def test_output_projection_and_residual(ctx, qtype):
    """attn_output.weight (896 x 896) applied to the attention output, then the
    residual add hidden += attn_out (tmac_gguf.cpp:1497-1499): the separate
    matmul + elem_op(0) and the fused tmac_matmul_add give the same bits."""
    rng = np.random.default_rng(61 + qtype)
    n = 896
    w = qwen_like(rng, qtype, n, n)
    ctxv = rng.standard_normal(n).astype(np.float32)
    hidden = rng.standard_normal(n).astype(np.float32)
    ref = oracle.matmul_q(qtype, w, ctxv, n, n)
    dw, dx, dy = ctx.upload(w), ctx.upload(ctxv), ctx.empty(n)
    ctx.matmul(qtype, n, n, dw, dx, dy)
    y = dy.numpy()
    assert_close(y, ref, "matmul")
    dh = ctx.upload(hidden)
    ctx.elem_op(0, dh, dy, n)  # separate residual add
    sep = dh.numpy()
    np.testing.assert_array_equal(sep, hidden + y)
    dh2 = ctx.upload(hidden)
    ctx.matmul(qtype, n, n, dw, dx, dh2, accumulate=True)  # fused
    np.testing.assert_array_equal(dh2.numpy(), sep)
    assert_close(dh2.numpy(), hidden + ref, "fused residual vs oracle")
    assert ctx.matmul(qtype, n, n, dw, dx, dx, check=False) == tmac_attn.TMAC_ERR_INVALID_ARG
    assert ctx.matmul(7, n, n, dw, dx, dy, accumulate=True, check=False) == tmac_attn.TMAC_ERR_UNSUPPORTED
    for d in (dw, dx, dy, dh, dh2):
        d.free()


def kquant_integer_blocks(rng, qtype, n):
    """Super-blocks whose weights are small integers (d = 1, unit scales), so
    integer inputs give exact sums in any order."""
    raw = rng.integers(0, 256, (n, oracle.BLOCK_BYTES[qtype]), dtype=np.uint8)
    one = np.frombuffer(np.float16(1).tobytes(), np.uint8)
    if qtype == oracle.Q6_K:
        raw[:, 208:210] = one
        raw[:, 192:208] = rng.integers(1, 4, (n, 16))  # int8 scales 1..3
    else:
        raw[:, 0:2] = one
        raw[:, 2:4] = one
    return raw.reshape(-1)


@pytest.mark.parametrize("qtype", [oracle.Q6_K, oracle.Q4_K])
@pytest.mark.parametrize("rows,cols", [(7, 256), (64, 4864), (129, 1024)])
def test_kquant_integer_pattern_bit_exact(ctx, qtype, rows, cols):
    rng = np.random.default_rng(120 + qtype + rows)
    w = kquant_integer_blocks(rng, qtype, rows * cols // 256)
    x = np.array([i % 7 - 3 for i in range(cols)], dtype=np.float32)
    dw, dx, dy = ctx.upload(w), ctx.upload(x), ctx.empty(rows)
    ctx.matmul(qtype, rows, cols, dw, dx, dy)
    np.testing.assert_array_equal(dy.numpy(), oracle.matmul_q(qtype, w, x, rows, cols))
    for d in (dw, dx, dy):
        d.free()


@pytest.mark.parametrize("qtype", [oracle.Q6_K, oracle.Q4_K])
def test_kquant_matmul_and_residual_match_oracle(ctx, qtype):
    """ffn_down shape (896 x 4864) with realistic scales; y = W x and y += W x."""
    rng = np.random.default_rng(130 + qtype)
    rows, cols = 896, 4864
    raw = rng.integers(0, 256, (rows * cols // 256, oracle.BLOCK_BYTES[qtype]), dtype=np.uint8)
    n = raw.shape[0]
    # super-block scales of a real checkpoint: d * sc (or d * scale) ~ 1e-3 .. 4e-3, |w| ~ 0.03
    sc = rng.uniform(2e-5, 6e-5, (n, 2)).astype(np.float16)
    if qtype == oracle.Q6_K:
        raw[:, 208:210] = sc[:, :1].view(np.uint8).reshape(n, 2)
    else:
        raw[:, 0:4] = sc.view(np.uint8).reshape(n, 4)
    w = raw.reshape(-1)
    x = rng.standard_normal(cols).astype(np.float32)
    h = rng.standard_normal(rows).astype(np.float32)
    ref = oracle.matmul_q(qtype, w, x, rows, cols)
    dw, dx, dy, dh = ctx.upload(w), ctx.upload(x), ctx.empty(rows), ctx.upload(h)
    ctx.matmul(qtype, rows, cols, dw, dx, dy)
    assert_close(dy.numpy(), ref, f"matmul type {qtype}")
    big = oracle.BLOCK_BYTES[qtype]
    wl = w.reshape(-1, big).copy()  # the same rows at 40x the scale: the order-independent bound
    sl = (sc.astype(np.float32) * 40).astype(np.float16)
    if qtype == oracle.Q6_K:
        wl[:, 208:210] = sl[:, :1].view(np.uint8).reshape(n, 2)
    else:
        wl[:, 0:4] = sl.view(np.uint8).reshape(n, 4)
    wl = wl.reshape(-1)
    dwl = ctx.upload(wl)
    ctx.matmul(qtype, rows, cols, dwl, dx, dy)
    refl = oracle.matmul_q(qtype, wl, x, rows, cols).astype(np.float64)
    wabs = np.stack([np.abs(np.array([oracle.dequant(qtype, wl, r * cols + c) for c in range(cols)]))
                     for r in range(0, rows, 97)])
    bound = 2 * (cols + 1) * 2.0 ** -24 * (wabs @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(dy.numpy().astype(np.float64)[::97] - refl[::97]) <= bound)
    dwl.free()
    ctx.matmul(qtype, rows, cols, dw, dx, dy)
    ctx.matmul(qtype, rows, cols, dw, dx, dh, accumulate=True)
    np.testing.assert_array_equal(dh.numpy(), h + dy.numpy())
    assert ctx.matmul(qtype, rows, 896, dw, dx, dy, check=False) == tmac_attn.TMAC_ERR_INVALID_ARG
    for d in (dw, dx, dy, dh):
        d.free()
