"""GPU parity of the whole attention block as one captured 24-layer step.

Per layer, as the reference's fused loop records it in one command buffer
(tmac_gguf.cpp:1478-1500, dispatches of metal_backend.hpp:456-489, 354-453,
320-338):
    fused_qkv_op + the three bias adds  ->  tmac_fused_qkv_bias
    rope_op x 2, elem_op(2) x 2, attention_op  ->  tmac_layer_attention_devpos
    attn_output matmul + residual elem_op(0)  ->  tmac_matmul_add (Q5_0 896 x 896)
then the position advance; 24 layers = 73 graph nodes, replayed for every
position 0..255 of zeroed caches.  Each layer reads its own normed input x_l
(synthetic: RMSNorm and the FFN between blocks are outside this path) and adds
its attention output into one hidden vector, as the reference's `hidden` is.

Oracle chain: oracle_qkv (tmac_gguf.cpp:1046-1081 + bias adds 1484-1489) ->
oracle_layer_step (990-1016, 1090-1091, 1093-1128) -> oracle_matmul_q (Q5_0,
510-514) + the residual add (1497-1499).  The projections are evaluated here in
numpy with the oracle's exact arithmetic (one fp32 accumulator per row, columns
ascending, each product rounded before the add; weights widened exactly), which
is checked bit for bit against the C oracle on the first step before it is
used for the sweep.  Every intermediate (q, k, v, the attention output) is held
to |gpu - ref| <= 2e-5 + 1e-4 |ref|, and so are the caches at the end (their
rows come from GPU and oracle projections that differ by rounding, so they are
not bit-identical).  The hidden vector is a sum of 25 terms of magnitude ~5
(the token's embedding and 24 projections) that often cancels to a small value,
so its bar is the same per-element rule applied to the magnitude of what was
added, |gpu - ref| <= 2e-5 + 1e-4 (|h0| + sum_l |y_l|): the fp32 allowance of
each term, summed.  Each decode step starts from a fresh embedding h0, as the
reference's `hidden` does for every token.
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close
from test_gpu_qkv import qwen_like
from test_oracle_quant import dequant_f64

pytestmark = pytest.mark.gpu
NH, NKV, HD = 14, 2, 64
QD, KVD = NH * HD, NKV * HD
NQKV = QD + 2 * KVD
W5_BYTES = lambda rows: rows * (QD // 32) * 22  # noqa: E731  Q5_0 bytes of rows x 896
W8_BYTES = lambda rows: rows * (QD // 32) * 34  # noqa: E731  Q8_0 bytes of rows x 896


def seq_gemv(wt: np.ndarray, x: np.ndarray) -> np.ndarray:
    """y[l][r] = sum_j w[l][r][j] x[l][j] with one fp32 accumulator per row, j ascending,
    each product rounded to fp32 before the add (the oracle's arithmetic); wt = [cols][L][rows]."""
    acc = np.zeros(wt.shape[1:], np.float32)
    for j in range(wt.shape[0]):
        acc = acc + wt[j] * x[:, j:j + 1]
    return acc


def block_weights(L: int, seed: int = 2024):
    rng = np.random.default_rng(seed)
    w = {"q": [], "k": [], "v": [], "o": [], "bq": [], "bk": [], "bv": []}
    for _ in range(L):
        w["q"].append(qwen_like(rng, oracle.Q5_0, QD, QD))
        w["k"].append(qwen_like(rng, oracle.Q5_0, KVD, QD))
        w["v"].append(qwen_like(rng, oracle.Q8_0, KVD, QD))
        w["o"].append(qwen_like(rng, oracle.Q5_0, QD, QD))
        w["bq"].append((rng.standard_normal(QD) * 0.1).astype(np.float32))
        w["bk"].append((rng.standard_normal(KVD) * 0.1).astype(np.float32))
        w["bv"].append((rng.standard_normal(KVD) * 0.1).astype(np.float32))
    return w


def test_attention_block_graph_sweep(ctx):
    L, cap = 24, 256
    w = block_weights(L)
    # dense fp32 weights (exact: d * q fits fp32), transposed for the column loop
    wqkv = np.stack([np.concatenate([dequant_f64(oracle.Q5_0, w["q"][l], QD, QD),
                                     dequant_f64(oracle.Q5_0, w["k"][l], KVD, QD),
                                     dequant_f64(oracle.Q8_0, w["v"][l], KVD, QD)]) for l in range(L)])
    wqkv_t = np.ascontiguousarray(wqkv.astype(np.float32).transpose(2, 0, 1))  # [896][L][1152]
    wo_t = np.ascontiguousarray(np.stack([dequant_f64(oracle.Q5_0, w["o"][l], QD, QD) for l in range(L)])
                                .astype(np.float32).transpose(2, 0, 1))     # [896][L][896]
    bias = np.stack([np.concatenate([w["bq"][l], w["bk"][l], w["bv"][l]]) for l in range(L)])
    xs = oracle.normal(3100, (cap, L, QD))          # the normed input of every layer at every step
    h0s = oracle.normal(3101, (cap, QD))            # each step's token embedding

    # device buffers: weight pools (layer l at l * matrix bytes), per-layer activations
    dwq = ctx.upload(np.concatenate(w["q"]))
    dwk = ctx.upload(np.concatenate(w["k"]))
    dwv = ctx.upload(np.concatenate(w["v"]))
    dwo = ctx.upload(np.concatenate(w["o"]))
    dbq, dbk, dbv = (ctx.upload(np.concatenate(w[b])) for b in ("bq", "bk", "bv"))
    dx = ctx.empty((L, QD))
    dq, dk, dv, dctx = ctx.empty((L, QD)), ctx.empty((L, KVD)), ctx.empty((L, KVD)), ctx.empty((L, QD))
    dh = ctx.empty(QD)
    kc = ctx.upload(np.zeros((L, cap, KVD), np.float32))
    vc = ctx.upload(np.zeros((L, cap, KVD), np.float32))
    pos = ctx.upload(np.zeros(1, np.int32))
    ctx.rope_prepare(HD, 1e6, cap)
    s = ctx.stream()
    ctx.step_begin(s)
    for l in range(L):
        ctx.fused_qkv(dwq.ptr + l * W5_BYTES(QD), dwk.ptr + l * W5_BYTES(KVD), dwv.ptr + l * W8_BYTES(KVD),
                      dx.at(l * QD), dq.at(l * QD), dk.at(l * KVD), dv.at(l * KVD), QD, KVD, KVD, QD, True,
                      b_q=dbq.at(l * QD), b_k=dbk.at(l * KVD), b_v=dbv.at(l * KVD), stream=s)
        ctx.layer_attention_devpos(dq.at(l * QD), dk.at(l * KVD), dv.at(l * KVD), kc.at(l * cap * KVD),
                                   vc.at(l * cap * KVD), dctx.at(l * QD), NH, NKV, HD, pos, cap, 1e6, stream=s)
        ctx.matmul(oracle.Q5_0, QD, QD, dwo.ptr + l * W5_BYTES(QD), dctx.at(l * QD), dh, accumulate=True, stream=s)
    ctx.pos_update(pos, 1, add=True, stream=s)
    g = ctx.step_end(s)

    ref_k = np.zeros((L, cap, KVD), np.float32)
    ref_v = np.zeros((L, cap, KVD), np.float32)
    try:
        for step in range(cap):
            dx.copy_from(xs[step])
            dh.copy_from(h0s[step])
            ctx.graph_launch(g, s)
            ctx.synchronize(s)
            # oracle chain
            qkv = seq_gemv(wqkv_t, xs[step]) + bias
            out = np.empty((L, QD), np.float32)
            for l in range(L):
                out[l], _, _ = oracle.layer_step(qkv[l, :QD], qkv[l, QD:QD + KVD], qkv[l, QD + KVD:], ref_k[l],
                                                 ref_v[l], NH, NKV, HD, step, 1e6)
            y = seq_gemv(wo_t, out)
            if step == 0:  # the numpy projections are the C oracle's, bit for bit
                for l in range(L):
                    rq, rk, rv = oracle.qkv(w["q"][l], w["k"][l], w["v"][l], True, xs[step, l], w["bq"][l],
                                            w["bk"][l], w["bv"][l], QD, KVD, KVD, QD)
                    np.testing.assert_array_equal(qkv[l], np.concatenate([rq, rk, rv]), err_msg=f"qkv layer {l}")
                    np.testing.assert_array_equal(y[l], oracle.matmul_q(oracle.Q5_0, w["o"][l], out[l], QD, QD))
            h, mag = h0s[step].copy(), np.abs(h0s[step]).astype(np.float64)
            for l in range(L):
                h = h + y[l]
                mag += np.abs(y[l])
            got_q, got_k, got_v = dq.numpy(), dk.numpy(), dv.numpy()
            got_ctx, got_h = dctx.numpy(), dh.numpy()
            assert_close(got_q, qkv[:, :QD], f"step {step}: q")
            assert_close(got_k, qkv[:, QD:QD + KVD], f"step {step}: k")
            assert_close(got_v, qkv[:, QD + KVD:], f"step {step}: v")
            assert_close(got_ctx, out, f"step {step}: attention output")
            err = np.abs(got_h.astype(np.float64) - h)
            assert np.all(err <= 2e-5 + 1e-4 * mag), \
                f"step {step}: hidden after 24 residual adds: max err {err.max():.3e}, worst margin " \
                f"{(err / (2e-5 + 1e-4 * mag)).max():.2f}"
        assert_close(kc.numpy(), ref_k, "k cache after the sweep")
        assert_close(vc.numpy(), ref_v, "v cache after the sweep")
        assert int(pos.numpy()[0]) == cap
    finally:
        ctx.graph_destroy(g)
        ctx.destroy_stream(s)
        for d in (dwq, dwk, dwv, dwo, dbq, dbk, dbv, dx, dq, dk, dv, dctx, dh, kc, vc, pos):
            d.free()
    assert ctx.check_device_error() == 0
