// test_layer_loop.cpp -- drives the attention slice of the reference's fused
// per-layer loop (tmac_gguf.cpp:1537-1568) through hip_backend, the C++
// mirror of metal_backend, and checks every layer of every step against the
// CPU oracle.  Prints PASS/FAIL per check like the reference's test_*.mm
// programs and exits non-zero on any failure.
//
// Per step (pos = 0..S-1), inside one batch_begin/batch_end:
//   for layer in 0..23:
//     producer: q_vec/k_new/v_new <- this layer's inputs (a device copy standing in
//               for fused_qkv_op + bias adds, tmac_gguf.cpp:1471-1489)
//     rope_op(q_vec, 14, 64, pos, 1e6); rope_op(k_new, 2, 64, pos, 1e6)     :1562-1563
//     elem_op(2, &k_cache[layer][pos][0], k_new, 128); elem_op(2, v ...)    :1564-1565
//     attention_op(q_vec, k_cache[layer], v_cache[layer], ctx[layer], 14, 2, 64, pos)  :1566-1568
// then the same step again through the fused layer_attention_op, compared too.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "tmac_hip_backend.hpp"
#include "tmac_oracle.h"

constexpr int L = 24, NH = 14, NKV = 2, HD = 64, KVD = NKV * HD, QD = NH * HD, CAP = 256;

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

int main(int argc, char** argv) {
    const int steps = argc > 1 ? std::atoi(argv[1]) : 6;
    hip_backend::Context mtl;
    if (!hip_backend::init(mtl, 0, 1000000.0f, CAP)) return 1;
    tmac_context* t = mtl.ctx;

    const size_t cache_f = (size_t)L * CAP * KVD;
    float *k_cache, *v_cache, *k2, *v2, *q_vec, *k_new, *v_new, *stage, *out, *out2;
    tmac_malloc(t, (void**)&k_cache, cache_f * 4);
    tmac_malloc(t, (void**)&v_cache, cache_f * 4);
    tmac_malloc(t, (void**)&k2, cache_f * 4);
    tmac_malloc(t, (void**)&v2, cache_f * 4);
    tmac_malloc(t, (void**)&q_vec, QD * 4);
    tmac_malloc(t, (void**)&k_new, KVD * 4);
    tmac_malloc(t, (void**)&v_new, KVD * 4);
    tmac_malloc(t, (void**)&stage, (size_t)L * (QD + 2 * KVD) * 4);
    tmac_malloc(t, (void**)&out, (size_t)L * QD * 4);
    tmac_malloc(t, (void**)&out2, (size_t)L * QD * 4);
    for (float* p : {k_cache, v_cache, k2, v2}) tmac_memset(t, mtl.stream, p, 0, cache_f * 4);  // reset_cache, :1430

    std::vector<float> ref_k(cache_f, 0.f), ref_v(cache_f, 0.f), host_stage((size_t)L * (QD + 2 * KVD));
    std::vector<float> got((size_t)L * QD), ref_out(QD), q(QD), kn(KVD);
    for (int pos = 0; pos < steps; pos++) {
        tmac_fill_normal(9000 + pos, host_stage.data(), host_stage.size());
        tmac_memcpy_h2d(t, mtl.stream, stage, host_stage.data(), host_stage.size() * 4);
        tmac_stream_synchronize(t, mtl.stream);

        hip_backend::batch_begin(mtl);
        for (int layer = 0; layer < L; layer++) {
            const float* s = stage + (size_t)layer * (QD + 2 * KVD);
            tmac_memcpy_d2d(t, mtl.stream, q_vec, s, QD * 4);
            tmac_memcpy_d2d(t, mtl.stream, k_new, s + QD, KVD * 4);
            tmac_memcpy_d2d(t, mtl.stream, v_new, s + QD + KVD, KVD * 4);
            float* kl = k_cache + (size_t)layer * CAP * KVD;
            float* vl = v_cache + (size_t)layer * CAP * KVD;
            hip_backend::rope_op(mtl, q_vec, NH, HD, pos, 1000000.0f);
            hip_backend::rope_op(mtl, k_new, NKV, HD, pos, 1000000.0f);
            hip_backend::elem_op(mtl, 2, kl + (size_t)pos * KVD, k_new, KVD);
            hip_backend::elem_op(mtl, 2, vl + (size_t)pos * KVD, v_new, KVD);
            hip_backend::attention_op(mtl, q_vec, kl, vl, out + (size_t)layer * QD, NH, NKV, HD, pos);
        }
        hip_backend::batch_end(mtl);
        check(mtl.last_status == TMAC_OK, "step recorded and ran", pos, 0);

        hip_backend::batch_begin(mtl);
        for (int layer = 0; layer < L; layer++) {
            const float* s = stage + (size_t)layer * (QD + 2 * KVD);
            hip_backend::layer_attention_op(mtl, s, s + QD, s + QD + KVD, k2 + (size_t)layer * CAP * KVD,
                                            v2 + (size_t)layer * CAP * KVD, out2 + (size_t)layer * QD, NH, NKV, HD,
                                            pos, CAP, 1000000.0f);
        }
        hip_backend::batch_end(mtl);
        check(mtl.last_status == TMAC_OK, "fused step recorded and ran", pos, 0);

        bool all_ok = true, all_ok2 = true;
        double worst = 0, worst2 = 0;
        tmac_memcpy_d2h(t, mtl.stream, got.data(), out, got.size() * 4);
        std::vector<float> got2((size_t)L * QD);
        tmac_memcpy_d2h(t, mtl.stream, got2.data(), out2, got2.size() * 4);
        tmac_stream_synchronize(t, mtl.stream);
        for (int layer = 0; layer < L; layer++) {
            const float* h = host_stage.data() + (size_t)layer * (QD + 2 * KVD);
            std::copy(h, h + QD, q.begin());
            std::copy(h + QD, h + QD + KVD, kn.begin());
            oracle_layer_step(q.data(), kn.data(), h + QD + KVD, ref_k.data() + (size_t)layer * CAP * KVD,
                              ref_v.data() + (size_t)layer * CAP * KVD, ref_out.data(), NH, NKV, HD, pos,
                              1000000.0f);
            bool ok;
            worst = std::fmax(worst, close_err(got.data() + (size_t)layer * QD, ref_out.data(), QD, &ok));
            all_ok &= ok;
            worst2 = std::fmax(worst2, close_err(got2.data() + (size_t)layer * QD, ref_out.data(), QD, &ok));
            all_ok2 &= ok;
        }
        check(all_ok, "per-op layer loop vs oracle", pos, worst);
        check(all_ok2, "fused layer loop vs oracle", pos, worst2);
    }
    std::vector<float> kc(cache_f), kc2(cache_f), vc(cache_f), vc2(cache_f);
    tmac_memcpy_d2h(t, mtl.stream, kc.data(), k_cache, cache_f * 4);
    tmac_memcpy_d2h(t, mtl.stream, vc.data(), v_cache, cache_f * 4);
    tmac_memcpy_d2h(t, mtl.stream, kc2.data(), k2, cache_f * 4);
    tmac_memcpy_d2h(t, mtl.stream, vc2.data(), v2, cache_f * 4);
    tmac_stream_synchronize(t, mtl.stream);
    check(kc == ref_k && vc == ref_v, "per-op caches bit-identical to oracle", steps, 0);
    check(kc2 == ref_k && vc2 == ref_v, "fused caches bit-identical to oracle", steps, 0);

    for (float* p : {k_cache, v_cache, k2, v2, q_vec, k_new, v_new, stage, out, out2}) tmac_free(t, p);
    hip_backend::shutdown(mtl);
    std::printf("%s (%d failures)\n", failures ? "FAIL" : "ALL PASS", failures);
    return failures ? 1 : 0;
}
