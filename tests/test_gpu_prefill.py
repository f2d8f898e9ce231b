"""GPU parity of the bf16-MFMA chunked causal prefill.

Oracle: the reference's decode applied per query row (tmac_gguf.cpp:1093-1128
with past_len = prefix + i), fed the bf16-rounded q/k/v the kernel computes
with (config 5 compares against the oracle on bf16-rounded
inputs).  Tolerance: the fp32 bound |gpu - ref| <= 2e-5 + 1e-4 |ref|.
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


def test_prefill_rejects_bad_arguments(ctx):
    import tmac_attn
    d = ctx.empty(16 * 14 * HD)
    assert ctx.prefill(d, d, d, d, 2, 16, 10, 20, 14, 2, HD, check=False) == tmac_attn.TMAC_ERR_INVALID_ARG
    assert ctx.prefill(d, d, d, d, 1, 16, 0, 16, 14, 2, 32, check=False) == tmac_attn.TMAC_ERR_UNSUPPORTED
    assert ctx.prefill(d, d, d, d, 1, 16, 0, 16, 14, 3, HD, check=False) == tmac_attn.TMAC_ERR_INVALID_ARG
