"""Seeded random sweeps of the path's smaller operators: the quantized GEMVs
(Q5_0, Q8_0, Q4_K, Q6_K; with and without the fused residual add), the fused
QKV projection with any subset of biases, RoPE over row ranges, elem_op copy
and add, and the KV-cache conversion.  Shapes are drawn at random, including
row counts that do not fill the last workgroup.

The GEMV cases use integer-valued weights (unit block scales) and inputs, so
every partial sum is an exact integer below 2^24 and the result must equal
the oracle (tmac_gguf.cpp:240-250, 311-327, 330-397, 510-514, 1046-1081) bit
for bit whatever the summation order; RoPE, the copy, the add and the
conversions are bit-exact by construction (tmac_gguf.cpp:990-1016,
kernel_elem.metal:19-20, extract_tmac.py:53-74).
"""
import numpy as np
import pytest

import oracle
import tmac_attn
from test_gpu_qkv import kquant_integer_blocks, q5_integer_pattern, run_qkv
from test_gpu_random_shapes import store
from test_oracle_quant import reference_q8_pattern

pytestmark = pytest.mark.gpu


def int_inputs(rng, n):
    return rng.integers(-3, 4, n).astype(np.float32)


@pytest.mark.parametrize("seed", range(24))
def test_random_gemv_integer_bit_exact(ctx, seed):
    rng = np.random.default_rng(11000 + seed)
    qtype = [oracle.Q5_0, oracle.Q8_0, oracle.Q4_K, oracle.Q6_K][seed % 4]
    rows = int(rng.choice([1, 3, 4, 5, int(rng.integers(6, 700))]))
    if qtype in (oracle.Q4_K, oracle.Q6_K):
        cols = 256 * int(rng.integers(1, 12))
        w = kquant_integer_blocks(rng, qtype, rows * cols // 256)
    else:
        cols = 32 * int(rng.integers(1, 80))
        w = (q5_integer_pattern(rows, cols, salt=seed)[0] if qtype == oracle.Q5_0
             else reference_q8_pattern(rows, cols)[0])
    x = int_inputs(rng, cols)
    hidden = int_inputs(rng, rows)
    what = f"seed {seed}: qtype={qtype} rows={rows} cols={cols}"
    dw, dx, dy, dh = ctx.upload(w), ctx.upload(x), ctx.empty(rows), ctx.upload(hidden)
    try:
        ref = oracle.matmul_q(qtype, w, x, rows, cols)
        ctx.matmul(qtype, rows, cols, dw, dx, dy)
        np.testing.assert_array_equal(dy.numpy(), ref, err_msg=what)
        ctx.matmul(qtype, rows, cols, dw, dx, dh, accumulate=True)  # y += W x
        np.testing.assert_array_equal(dh.numpy(), hidden + ref, err_msg=what + " (residual)")
    finally:
        for d in (dw, dx, dy, dh):
            d.free()


@pytest.mark.parametrize("seed", range(16))
def test_random_qkv_integer_bit_exact(ctx, seed):
    rng = np.random.default_rng(11100 + seed)
    cols = 32 * int(rng.integers(1, 40))
    nq, nk, nv = (int(rng.integers(0, 200)) for _ in range(3))
    if nq + nk + nv == 0:
        nq = 1
    v_is_q8 = bool(rng.integers(0, 2))
    wq = q5_integer_pattern(nq, cols, salt=seed)[0] if nq else None
    wk = q5_integer_pattern(nk, cols, salt=seed + 1)[0] if nk else None
    wv = (reference_q8_pattern(nv, cols)[0] if v_is_q8 else q5_integer_pattern(nv, cols, salt=seed + 2)[0]) \
        if nv else None
    x = int_inputs(rng, cols)
    bias = tuple(int_inputs(rng, n) if (n and rng.random() < 0.6) else None for n in (nq, nk, nv))
    what = f"seed {seed}: cols={cols} rows={nq}/{nk}/{nv} v_is_q8={v_is_q8} bias={[b is not None for b in bias]}"
    got = run_qkv(ctx, wq, wk, wv, x, nq, nk, nv, cols, v_is_q8, bias)
    ref = oracle.qkv(wq if nq else np.zeros(0, np.uint8), wk if nk else np.zeros(0, np.uint8),
                     wv if nv else np.zeros(0, np.uint8), v_is_q8, x, *bias, nq, nk, nv, cols)
    for g, r, name in zip(got, ref, "qkv"):
        np.testing.assert_array_equal(g, r, err_msg=f"{what}: {name}")


@pytest.mark.parametrize("seed", range(16))
def test_random_rope_rows_bit_exact(ctx, seed):
    """RoPE on n_rows rows at positions first_pos .. first_pos + n_rows - 1, rows
    row_stride floats apart (the floats between rows are left alone); a stride that
    leaves rows off 16-byte alignment is refused before any launch."""
    rng = np.random.default_rng(11200 + seed)
    n_heads = int(rng.integers(1, 17))
    hd = int(rng.choice([2, 8, 32, 64, 64, 96, 128, 256]))
    n_rows = int(rng.integers(1, 40))
    natural = n_heads * hd
    stride = (natural + 3) // 4 * 4 + int(rng.choice([0, 0, 4, 64]))  # rows 16-byte aligned
    first = int(rng.choice([0, int(rng.integers(1, 100)), int(rng.integers(100, 30000))]))
    base = float(rng.choice([1e4, 1e6]))
    x = oracle.normal(11300 + seed, n_rows * stride)
    dx = ctx.upload(x)
    try:
        if natural % 4:  # a row stride that is not 16-byte aligned is refused
            with pytest.raises(tmac_attn.TmacError) as e:
                ctx.rope_rows(dx, n_rows, natural, n_heads, hd, first, base)
            assert e.value.status == tmac_attn.TMAC_ERR_MISALIGNED
        ctx.rope_rows(dx, n_rows, stride, n_heads, hd, first, base)
        got = dx.numpy()
    finally:
        dx.free()
    ref = x.copy()
    for r in range(n_rows):
        row = slice(r * stride, r * stride + n_heads * hd)
        ref[row] = oracle.rope_heads(x[row], n_heads, hd, first + r, base)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32),
                                  err_msg=f"seed {seed}: heads={n_heads} hd={hd} rows={n_rows} stride={stride} "
                                          f"first={first} base={base}")


@pytest.mark.parametrize("seed", range(12))
def test_random_elem_ops_bit_exact(ctx, seed):
    """elem_op 2 (the cache write: data = aux) and 0 (data += aux) on any length."""
    rng = np.random.default_rng(11400 + seed)
    dim = int(rng.choice([1, 2, 3, 63, 64, 65, 128, int(rng.integers(129, 20000))]))
    a, b = oracle.normal(11500 + seed, dim), oracle.normal(11501 + seed, dim)
    da, db = ctx.upload(a), ctx.upload(b)
    try:
        ctx.elem_op(0, da, db, dim)
        np.testing.assert_array_equal(da.numpy(), a + b, err_msg=f"add dim={dim}")
        ctx.elem_op(2, da, db, dim)
        np.testing.assert_array_equal(da.numpy().view(np.uint32), b.view(np.uint32), err_msg=f"copy dim={dim}")
    finally:
        da.free()
        db.free()


@pytest.mark.parametrize("seed", range(12))
def test_random_kv_convert_bit_exact(ctx, seed):
    """fp32 rows to the bf16, fp16 and Q8_0 cache formats, any multiple of 64 values,
    rows of very different magnitudes."""
    rng = np.random.default_rng(11600 + seed)
    dt = [tmac_attn.TMAC_KV_BF16, tmac_attn.TMAC_KV_F16, tmac_attn.TMAC_KV_Q8_0][seed % 3]
    n = 64 * int(rng.integers(1, 3000))
    x = oracle.normal(11700 + seed, (n // 64, 64))
    x *= np.exp2(rng.uniform(-8, 8, (n // 64, 1))).astype(np.float32)
    ref = store(x.reshape(-1, 64), dt, 1)
    dx = ctx.upload(x)
    dy = ctx.empty(ref.shape, ref.dtype)
    try:
        ctx.kv_convert(dt, dx, dy, n)
        np.testing.assert_array_equal(dy.numpy(), ref, err_msg=f"seed {seed}: dt={dt} n={n}")
    finally:
        dx.free()
        dy.free()
