// test_layer_loop.cpp -- drives the attention block of the reference's fused
// per-layer loop (tmac_gguf.cpp:1466-1500) through hip_backend, the C++
// mirror of metal_backend, and checks every layer of every step against the
// CPU oracle.  Prints PASS/FAIL per check like the reference's test_*.mm
// programs and exits non-zero on any failure.
//
// Per step (pos = 0..S-1), inside one batch_begin/batch_end, for layer 0..23
// (x = the layer's normed input; RMSNorm and the FFN are outside this path):
//   fused_qkv_op(Wq, Wk, Wv, x -> q_vec, k_new, v_new)                     :1478-1482
//   elem_op(0, q_vec, bq, 896); elem_op(0, k_new, bk, 128); elem_op(0, v_new, bv, 128)   :1483-1489
//   rope_op(q_vec, 14, 64, pos, 1e6); rope_op(k_new, 2, 64, pos, 1e6)     :1490-1491
//   elem_op(2, &k_cache[layer][pos][0], k_new, 128); elem_op(2, v ...)    :1492-1493
//   attention_op(q_vec, k_cache[layer], v_cache[layer], context, 14, 2, 64, pos)  :1494-1496
//   matmul(attn_output, context -> attn_out); elem_op(0, hidden, attn_out, 896)  :1497-1499
// then the same step again through the fused entry points (fused_qkv_bias_op,
// layer_attention_op, matmul_add_op) on caches and a hidden vector of its own.
//
// Checks per layer and step: the projections (q, k, v after the biases) against
// oracle_qkv; both paths' attention outputs against oracle_layer_step fed the
// GPU's own q, k, v (so the cache rows, written from them, stay bit-identical to
// the oracle's); the hidden vector after every step against oracle_matmul_q plus
// the residual add, both paths, from a fresh token embedding every step (the
// reference's `hidden` per token).  The hidden vector sums 25 terms of magnitude
// ~5 that often cancel, so it is held to the fp32 rule on the magnitude of what
// was added, |gpu - ref| <= 2e-5 + 1e-4 (|h0| + sum_l |y_l|).  The per-op q, k
// and v must equal the fused path's bit for bit (the fused bias adds round as
// the separate adds do).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "tmac_hip_backend.hpp"
#include "tmac_oracle.h"

constexpr int L = 24, NH = 14, NKV = 2, HD = 64, KVD = NKV * HD, QD = NH * HD, CAP = 256;
constexpr int NB = QD / 32;                                   // blocks per weight row (896 inputs)
constexpr size_t WQ = (size_t)QD * NB * 22, WK = (size_t)KVD * NB * 22, WV = (size_t)KVD * NB * 34;
constexpr size_t WO = WQ;                                     // attn_output: Q5_0 896 x 896

static int failures = 0;

static void check(bool ok, const char* what, int step, double err) {
    std::printf("%s: %s step %d (max err %.3g)\n", ok ? "PASS" : "FAIL", what, step, err);
    if (!ok) failures++;
}

static double close_err(const float* got, const float* ref, size_t n, bool* ok) {
    double worst = 0;
    *ok = true;
    for (size_t i = 0; i < n; i++) {
        double e = std::fabs((double)got[i] - ref[i]);
        if (!(e <= 2e-5 + 1e-4 * std::fabs((double)ref[i]))) *ok = false;
        if (e > worst || std::isnan(e)) worst = e;
    }
    return worst;
}

// GGML Q5_0 / Q8_0 blocks with random codes and fp16 scales of +-[2^-9, 2^-8)
// (the magnitudes of a Q5_0 Qwen2-0.5B checkpoint), from a xorshift stream.
static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint32_t next_u32() {
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return (uint32_t)(rng_state >> 16);
}
static void fill_blocks(std::vector<uint8_t>& w, size_t n_blocks, int block_bytes) {
    w.resize(n_blocks * block_bytes);
    for (size_t b = 0; b < n_blocks; b++) {
        uint8_t* p = w.data() + b * block_bytes;
        const uint16_t d = (uint16_t)(0x1800u | (next_u32() & 0x3FFu) | ((next_u32() & 1u) << 15));
        p[0] = (uint8_t)(d & 0xFF);
        p[1] = (uint8_t)(d >> 8);
        for (int i = 2; i < block_bytes; i++) p[i] = (uint8_t)next_u32();
    }
}

int main(int argc, char** argv) {
    const int steps = argc > 1 ? std::atoi(argv[1]) : 6;
    hip_backend::Context mtl;
    if (!hip_backend::init(mtl, 0, 1000000.0f, CAP)) return 1;
    tmac_context* t = mtl.ctx;

    // weights and biases of every layer, on the host and in one device pool each
    std::vector<uint8_t> hwq, hwk, hwv, hwo;
    fill_blocks(hwq, (size_t)L * QD * NB, 22);
    fill_blocks(hwk, (size_t)L * KVD * NB, 22);
    fill_blocks(hwv, (size_t)L * KVD * NB, 34);
    fill_blocks(hwo, (size_t)L * QD * NB, 22);
    std::vector<float> hb((size_t)L * (QD + 2 * KVD));
    tmac_fill_normal(8800, hb.data(), hb.size());
    for (float& b : hb) b *= 0.1f;
    uint8_t *wq, *wk, *wv, *wo;
    float* bias;
    tmac_malloc(t, (void**)&wq, hwq.size());
    tmac_malloc(t, (void**)&wk, hwk.size());
    tmac_malloc(t, (void**)&wv, hwv.size());
    tmac_malloc(t, (void**)&wo, hwo.size());
    tmac_malloc(t, (void**)&bias, hb.size() * 4);
    tmac_memcpy_h2d(t, mtl.stream, wq, hwq.data(), hwq.size());
    tmac_memcpy_h2d(t, mtl.stream, wk, hwk.data(), hwk.size());
    tmac_memcpy_h2d(t, mtl.stream, wv, hwv.data(), hwv.size());
    tmac_memcpy_h2d(t, mtl.stream, wo, hwo.data(), hwo.size());
    tmac_memcpy_h2d(t, mtl.stream, bias, hb.data(), hb.size() * 4);
    auto bq = [&](int l) { return bias + (size_t)l * (QD + 2 * KVD); };
    auto bk = [&](int l) { return bq(l) + QD; };
    auto bv = [&](int l) { return bq(l) + QD + KVD; };

    const size_t cache_f = (size_t)L * CAP * KVD;
    float *k_cache, *v_cache, *k2, *v2, *x, *qkv, *qkv2, *ctx, *ctx2, *attn_out, *hidden, *hidden2;
    tmac_malloc(t, (void**)&k_cache, cache_f * 4);
    tmac_malloc(t, (void**)&v_cache, cache_f * 4);
    tmac_malloc(t, (void**)&k2, cache_f * 4);
    tmac_malloc(t, (void**)&v2, cache_f * 4);
    tmac_malloc(t, (void**)&x, (size_t)L * QD * 4);
    tmac_malloc(t, (void**)&qkv, (size_t)L * (QD + 2 * KVD) * 4);   // per layer: q_vec, k_new, v_new
    tmac_malloc(t, (void**)&qkv2, (size_t)L * (QD + 2 * KVD) * 4);
    tmac_malloc(t, (void**)&ctx, (size_t)L * QD * 4);
    tmac_malloc(t, (void**)&ctx2, (size_t)L * QD * 4);
    tmac_malloc(t, (void**)&attn_out, (size_t)L * QD * 4);
    tmac_malloc(t, (void**)&hidden, QD * 4);
    tmac_malloc(t, (void**)&hidden2, QD * 4);
    for (float* p : {k_cache, v_cache, k2, v2}) tmac_memset(t, mtl.stream, p, 0, cache_f * 4);  // reset_cache, :1430
    std::vector<float> ref_h(QD);
    std::vector<double> mag(QD);

    std::vector<float> ref_k(cache_f, 0.f), ref_v(cache_f, 0.f), hx((size_t)L * QD);
    std::vector<float> g_qkv((size_t)L * (QD + 2 * KVD)), g_qkv2(g_qkv.size()), g_ctx((size_t)L * QD),
        g_ctx2(g_ctx.size()), g_h(QD), g_h2(QD), rq(QD), rk(KVD), rv(KVD), ro(QD), ry(QD), q(QD), kn(KVD);
    for (int pos = 0; pos < steps; pos++) {
        tmac_fill_normal(9000 + pos, hx.data(), hx.size());
        tmac_memcpy_h2d(t, mtl.stream, x, hx.data(), hx.size() * 4);
        tmac_fill_normal(8900 + pos, ref_h.data(), QD);  // this token's embedding
        tmac_memcpy_h2d(t, mtl.stream, hidden, ref_h.data(), QD * 4);
        tmac_memcpy_h2d(t, mtl.stream, hidden2, ref_h.data(), QD * 4);
        for (int i = 0; i < QD; i++) mag[i] = std::fabs((double)ref_h[i]);
        tmac_stream_synchronize(t, mtl.stream);

        hip_backend::batch_begin(mtl);
        for (int layer = 0; layer < L; layer++) {
            float* q_vec = qkv + (size_t)layer * (QD + 2 * KVD);
            float* k_new = q_vec + QD;
            float* v_new = k_new + KVD;
            float* kl = k_cache + (size_t)layer * CAP * KVD;
            float* vl = v_cache + (size_t)layer * CAP * KVD;
            float* c = ctx + (size_t)layer * QD;
            hip_backend::fused_qkv_op(mtl, wq + layer * WQ, wk + layer * WK, wv + layer * WV, x + (size_t)layer * QD,
                                      q_vec, k_new, v_new, QD, KVD, KVD, QD, true);
            hip_backend::elem_op(mtl, 0, q_vec, bq(layer), QD);
            hip_backend::elem_op(mtl, 0, k_new, bk(layer), KVD);
            hip_backend::elem_op(mtl, 0, v_new, bv(layer), KVD);
            hip_backend::rope_op(mtl, q_vec, NH, HD, pos, 1000000.0f);
            hip_backend::rope_op(mtl, k_new, NKV, HD, pos, 1000000.0f);
            hip_backend::elem_op(mtl, 2, kl + (size_t)pos * KVD, k_new, KVD);
            hip_backend::elem_op(mtl, 2, vl + (size_t)pos * KVD, v_new, KVD);
            hip_backend::attention_op(mtl, q_vec, kl, vl, c, NH, NKV, HD, pos);
            hip_backend::matmul_q5_0(mtl, QD, QD, wo + layer * WO, c, attn_out + (size_t)layer * QD);
            hip_backend::elem_op(mtl, 0, hidden, attn_out + (size_t)layer * QD, QD);
        }
        hip_backend::batch_end(mtl);
        check(mtl.last_status == TMAC_OK, "step recorded and ran", pos, 0);

        hip_backend::batch_begin(mtl);
        for (int layer = 0; layer < L; layer++) {
            float* q_vec = qkv2 + (size_t)layer * (QD + 2 * KVD);
            float* c = ctx2 + (size_t)layer * QD;
            hip_backend::fused_qkv_bias_op(mtl, wq + layer * WQ, wk + layer * WK, wv + layer * WV,
                                           x + (size_t)layer * QD, bq(layer), bk(layer), bv(layer), q_vec,
                                           q_vec + QD, q_vec + QD + KVD, QD, KVD, KVD, QD, true);
            hip_backend::layer_attention_op(mtl, q_vec, q_vec + QD, q_vec + QD + KVD, k2 + (size_t)layer * CAP * KVD,
                                            v2 + (size_t)layer * CAP * KVD, c, NH, NKV, HD, pos, CAP, 1000000.0f);
            hip_backend::matmul_add_op(mtl, TMAC_Q5_0, QD, QD, wo + layer * WO, c, hidden2);
        }
        hip_backend::batch_end(mtl);
        check(mtl.last_status == TMAC_OK, "fused step recorded and ran", pos, 0);

        tmac_memcpy_d2h(t, mtl.stream, g_qkv.data(), qkv, g_qkv.size() * 4);
        tmac_memcpy_d2h(t, mtl.stream, g_qkv2.data(), qkv2, g_qkv2.size() * 4);
        tmac_memcpy_d2h(t, mtl.stream, g_ctx.data(), ctx, g_ctx.size() * 4);
        tmac_memcpy_d2h(t, mtl.stream, g_ctx2.data(), ctx2, g_ctx2.size() * 4);
        tmac_memcpy_d2h(t, mtl.stream, g_h.data(), hidden, QD * 4);
        tmac_memcpy_d2h(t, mtl.stream, g_h2.data(), hidden2, QD * 4);
        tmac_stream_synchronize(t, mtl.stream);
        bool ok_p = true, ok_a = true, ok_a2 = true, same_rope = true;
        double w_p = 0, w_a = 0, w_a2 = 0;
        for (int layer = 0; layer < L; layer++) {
            const float* g2 = g_qkv2.data() + (size_t)layer * (QD + 2 * KVD);  // pre-RoPE q, k (fused path)
            const float* g1 = g_qkv.data() + (size_t)layer * (QD + 2 * KVD);   // RoPE'd q, k (per-op path)
            oracle_qkv(hwq.data() + layer * WQ, hwk.data() + layer * WK, hwv.data() + layer * WV, 1,
                       hx.data() + (size_t)layer * QD, hb.data() + (size_t)layer * (QD + 2 * KVD),
                       hb.data() + (size_t)layer * (QD + 2 * KVD) + QD,
                       hb.data() + (size_t)layer * (QD + 2 * KVD) + QD + KVD, rq.data(), rk.data(), rv.data(), QD, KVD,
                       KVD, QD);
            bool ok;
            w_p = std::fmax(w_p, close_err(g2, rq.data(), QD, &ok));
            ok_p &= ok;
            w_p = std::fmax(w_p, close_err(g2 + QD, rk.data(), KVD, &ok));
            ok_p &= ok;
            w_p = std::fmax(w_p, close_err(g2 + QD + KVD, rv.data(), KVD, &ok));
            ok_p &= ok;
            for (int i = 0; i < KVD; i++) same_rope &= g1[QD + KVD + i] == g2[QD + KVD + i];  // v: never rotated
            // the attention slice on the GPU's own projections
            std::copy(g2, g2 + QD, q.begin());
            std::copy(g2 + QD, g2 + QD + KVD, kn.begin());
            oracle_layer_step(q.data(), kn.data(), g2 + QD + KVD, ref_k.data() + (size_t)layer * CAP * KVD,
                              ref_v.data() + (size_t)layer * CAP * KVD, ro.data(), NH, NKV, HD, pos, 1000000.0f);
            // the per-op path's rope_op results equal the oracle's RoPE of the same projections
            for (int i = 0; i < QD; i++) same_rope &= g1[i] == q[i];
            for (int i = 0; i < KVD; i++) same_rope &= g1[QD + i] == kn[i];
            w_a = std::fmax(w_a, close_err(g_ctx.data() + (size_t)layer * QD, ro.data(), QD, &ok));
            ok_a &= ok;
            w_a2 = std::fmax(w_a2, close_err(g_ctx2.data() + (size_t)layer * QD, ro.data(), QD, &ok));
            ok_a2 &= ok;
            // output projection of the fused path's attention output, then the residual add
            oracle_matmul_q(TMAC_Q5_0, hwo.data() + layer * WO, g_ctx2.data() + (size_t)layer * QD, ry.data(), QD, QD);
            for (int i = 0; i < QD; i++) {
                ref_h[i] = ref_h[i] + ry[i];
                mag[i] += std::fabs((double)ry[i]);
            }
        }
        check(ok_p, "QKV projections + biases vs oracle", pos, w_p);
        check(same_rope, "per-op projections equal the fused ones, RoPE'd q and k equal to the oracle's", pos, 0);
        check(ok_a, "per-op attention vs oracle", pos, w_a);
        check(ok_a2, "fused attention vs oracle", pos, w_a2);
        bool ok_h = true, ok_h2 = true;
        double w_h = 0, w_h2 = 0;
        for (int i = 0; i < QD; i++) {
            const double bar = 2e-5 + 1e-4 * mag[i];
            const double e1 = std::fabs((double)g_h[i] - ref_h[i]), e2 = std::fabs((double)g_h2[i] - ref_h[i]);
            ok_h &= e1 <= bar;
            ok_h2 &= e2 <= bar;
            w_h = std::fmax(w_h, e1);
            w_h2 = std::fmax(w_h2, e2);
        }
        check(ok_h, "per-op hidden after 24 output projections + residual adds vs oracle", pos, w_h);
        check(ok_h2, "fused hidden after 24 output projections + residual adds vs oracle", pos, w_h2);
    }
    std::vector<float> kc(cache_f), kc2(cache_f), vc(cache_f), vc2(cache_f);
    tmac_memcpy_d2h(t, mtl.stream, kc.data(), k_cache, cache_f * 4);
    tmac_memcpy_d2h(t, mtl.stream, vc.data(), v_cache, cache_f * 4);
    tmac_memcpy_d2h(t, mtl.stream, kc2.data(), k2, cache_f * 4);
    tmac_memcpy_d2h(t, mtl.stream, vc2.data(), v2, cache_f * 4);
    tmac_stream_synchronize(t, mtl.stream);
    check(kc == ref_k && vc == ref_v, "per-op caches bit-identical to oracle", steps, 0);
    check(kc2 == ref_k && vc2 == ref_v, "fused caches bit-identical to oracle", steps, 0);

    for (void* p : {(void*)k_cache, (void*)v_cache, (void*)k2, (void*)v2, (void*)x, (void*)qkv, (void*)qkv2,
                    (void*)ctx, (void*)ctx2, (void*)attn_out, (void*)hidden, (void*)hidden2, (void*)wq, (void*)wk,
                    (void*)wv, (void*)wo, (void*)bias})
        tmac_free(t, p);
    hip_backend::shutdown(mtl);
    std::printf("%s (%d failures)\n", failures ? "FAIL" : "ALL PASS", failures);
    return failures ? 1 : 0;
}
