// test_paged_serving.cpp -- a serving loop over paged Q8_0 KV caches, driven
// through the C ABI (include/tmac_attn.h) the way an engine would drive it:
// n_seq sequences at different positions share per-layer page pools through
// one block table (pages in random pool order), and every decode step is one
// captured graph of tmac_layer_attention_paged calls (one per layer), replayed
// with new inputs and new device-side positions.  Checked against the CPU
// oracle: per layer and sequence, RoPE (tmac_gguf.cpp:990-1016), the new row
// quantized to Q8_0 with the reference converter's rule
// (scripts/extract_tmac.py:159-173) and written at its position
// (tmac_gguf.cpp:1090-1091), then attention over the widened rows
// (tmac_gguf.cpp:1093-1128); at the end every pool byte is compared.  Prints
// PASS/FAIL per check and exits non-zero on any failure.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <numeric>
#include <random>
#include <vector>

#include "tmac_attn.h"
#include "tmac_oracle.h"

constexpr int L = 4, NH = 14, NKV = 2, HD = 64, KVD = NKV * HD, QD = NH * HD;
constexpr int HB = 68, ROWB = NKV * HB, PR = 16;  // Q8_0 head row bytes, cache row bytes, rows per page

static int failures = 0;

static void check(bool ok, const char* what, int step, double err) {
    std::printf("%s: %s step %d (max err %.3g)\n", ok ? "PASS" : "FAIL", what, step, err);
    if (!ok) failures++;
}

#define ABI(call)                                                                              \
    do {                                                                                       \
        int rc_ = (call);                                                                      \
        if (rc_ != TMAC_OK) {                                                                  \
            std::printf("FAIL: %s -> %s (%s)\n", #call, tmac_status_string(rc_), tmac_last_error(t)); \
            return 1;                                                                          \
        }                                                                                      \
    } while (0)

int main(int argc, char** argv) {
    const int steps = argc > 1 ? std::atoi(argv[1]) : 5;
    tmac_context* t = nullptr;
    if (tmac_init(&t, 0) != TMAC_OK) {
        std::printf("FAIL: tmac_init\n");
        return 1;
    }
    tmac_stream s = nullptr;
    ABI(tmac_stream_create(t, &s));

    const std::vector<int> pos0 = {0, 5, 17, 300, 1023, 63};
    const int n_seq = (int)pos0.size();
    const int last = *std::max_element(pos0.begin(), pos0.end()) + steps;  // highest position written
    const int max_pages = last / PR + 1;
    const int max_len = max_pages * PR;

    // Block table: each sequence's logical pages on distinct pool pages, in random order.
    std::vector<int> need(n_seq);
    for (int q = 0; q < n_seq; q++) need[q] = (pos0[q] + steps - 1) / PR + 1;
    const int n_pages = std::accumulate(need.begin(), need.end(), 0) + 9;
    std::vector<int> perm(n_pages);
    std::iota(perm.begin(), perm.end(), 0);
    std::shuffle(perm.begin(), perm.end(), std::mt19937(11));
    std::vector<int32_t> table((size_t)n_seq * max_pages, 0);
    for (int q = 0, nxt = 0; q < n_seq; q++)
        for (int j = 0; j < need[q]; j++) table[(size_t)q * max_pages + j] = perm[nxt++];

    // Reference caches: per layer and sequence, dense Q8_0 rows; rows below the start
    // position hold quantized N(0,1) rows, the rest are zero.
    std::vector<uint8_t> dk((size_t)L * n_seq * max_len * ROWB, 0), dv(dk.size(), 0);
    auto drow = [&](std::vector<uint8_t>& d, int l, int q, int r) {
        return d.data() + (((size_t)l * n_seq + q) * max_len + r) * ROWB;
    };
    std::vector<float> tmp((size_t)1100 * KVD);
    for (int l = 0; l < L; l++)
        for (int q = 0; q < n_seq; q++)
            if (pos0[q] > 0) {
                tmac_fill_normal(5000 + 10 * l + q, tmp.data(), (size_t)pos0[q] * KVD);
                oracle_q8_kv_rows(tmp.data(), (int64_t)pos0[q] * NKV, drow(dk, l, q, 0));
                tmac_fill_normal(6000 + 10 * l + q, tmp.data(), (size_t)pos0[q] * KVD);
                oracle_q8_kv_rows(tmp.data(), (int64_t)pos0[q] * NKV, drow(dv, l, q, 0));
            }
    const size_t pool_b = (size_t)n_pages * PR * ROWB;
    auto scatter = [&](const std::vector<uint8_t>& d, int l) {  // dense rows -> the pool through the table
        std::vector<uint8_t> pool(pool_b, 0);
        for (int q = 0; q < n_seq; q++)
            for (int r = 0; r < need[q] * PR; r++) {
                const size_t prow = (size_t)table[(size_t)q * max_pages + r / PR] * PR + r % PR;
                std::memcpy(pool.data() + prow * ROWB, d.data() + (((size_t)l * n_seq + q) * max_len + r) * ROWB,
                            ROWB);
            }
        return pool;
    };

    // Device buffers.
    std::vector<void*> kp(L), vp(L);
    for (int l = 0; l < L; l++) {
        ABI(tmac_malloc(t, &kp[l], pool_b));
        ABI(tmac_malloc(t, &vp[l], pool_b));
        const std::vector<uint8_t> hk = scatter(dk, l), hv = scatter(dv, l);
        ABI(tmac_memcpy_h2d(t, s, kp[l], hk.data(), pool_b));
        ABI(tmac_memcpy_h2d(t, s, vp[l], hv.data(), pool_b));
    }
    int32_t *d_table, *d_pos;
    float *d_q, *d_kn, *d_vn, *d_out;
    const size_t qn = (size_t)L * n_seq * QD, kn = (size_t)L * n_seq * KVD;
    ABI(tmac_malloc(t, (void**)&d_table, table.size() * 4));
    ABI(tmac_malloc(t, (void**)&d_pos, (size_t)n_seq * 4));
    ABI(tmac_malloc(t, (void**)&d_q, qn * 4));
    ABI(tmac_malloc(t, (void**)&d_kn, kn * 4));
    ABI(tmac_malloc(t, (void**)&d_vn, kn * 4));
    ABI(tmac_malloc(t, (void**)&d_out, qn * 4));
    ABI(tmac_memcpy_h2d(t, s, d_table, table.data(), table.size() * 4));
    ABI(tmac_memcpy_h2d(t, s, d_pos, pos0.data(), (size_t)n_seq * 4));
    for (float* p : {d_q, d_kn, d_vn}) ABI(tmac_memset(t, s, p, 0, (p == d_q ? qn : kn) * 4));
    ABI(tmac_rope_prepare(t, HD, 1000000.0f, max_len));

    auto layer_calls = [&]() {
        for (int l = 0; l < L; l++) {
            const int rc = tmac_layer_attention_paged(
                t, s, TMAC_KV_Q8_0, d_q + (size_t)l * n_seq * QD, d_kn + (size_t)l * n_seq * KVD,
                d_vn + (size_t)l * n_seq * KVD, kp[l], vp[l], n_pages, d_table, max_pages, d_pos,
                d_out + (size_t)l * n_seq * QD, n_seq, NH, NKV, HD, max_len, 1000000.0f);
            if (rc != TMAC_OK) return rc;
        }
        return (int)TMAC_OK;
    };
    // One eager pass sizes the split workspace outside capture; it writes row pos0 of
    // every sequence from zero inputs, which the first replay (same positions) rewrites.
    ABI(layer_calls());
    ABI(tmac_stream_synchronize(t, s));
    ABI(tmac_step_begin(t, s));
    const int rc_cap = layer_calls();
    tmac_graph* g = nullptr;
    ABI(tmac_step_end(t, s, &g));
    ABI(rc_cap);

    std::vector<float> hq(qn), hk(kn), hv(kn), got(qn), ref(QD), kw((size_t)max_len * KVD), vw(kw.size());
    std::vector<int> pos(pos0);
    for (int step = 0; step < steps; step++) {
        tmac_fill_normal(7000 + step, hq.data(), qn);
        tmac_fill_normal(8000 + step, hk.data(), kn);
        tmac_fill_normal(9000 + step, hv.data(), kn);
        ABI(tmac_memcpy_h2d(t, s, d_q, hq.data(), qn * 4));
        ABI(tmac_memcpy_h2d(t, s, d_kn, hk.data(), kn * 4));
        ABI(tmac_memcpy_h2d(t, s, d_vn, hv.data(), kn * 4));
        ABI(tmac_memcpy_h2d(t, s, d_pos, pos.data(), (size_t)n_seq * 4));
        ABI(tmac_graph_launch(t, g, s));
        ABI(tmac_memcpy_d2h(t, s, got.data(), d_out, qn * 4));
        ABI(tmac_stream_synchronize(t, s));

        bool ok = true;
        double worst = 0;
        for (int l = 0; l < L; l++)
            for (int q = 0; q < n_seq; q++) {
                const size_t qo = ((size_t)l * n_seq + q) * QD, ko = ((size_t)l * n_seq + q) * KVD;
                float* qq = hq.data() + qo;
                float* kk = hk.data() + ko;
                oracle_rope(qq, kk, NH, NKV, HD, pos[q], 1000000.0f);
                oracle_q8_kv_rows(kk, NKV, drow(dk, l, q, pos[q]));
                oracle_q8_kv_rows(hv.data() + ko, NKV, drow(dv, l, q, pos[q]));
                oracle_q8_kv_widen(drow(dk, l, q, 0), (int64_t)(pos[q] + 1) * NKV, kw.data());
                oracle_q8_kv_widen(drow(dv, l, q, 0), (int64_t)(pos[q] + 1) * NKV, vw.data());
                oracle_attention(qq, kw.data(), vw.data(), ref.data(), NH, NKV, HD, pos[q]);
                for (int i = 0; i < QD; i++) {
                    const double e = std::fabs((double)got[qo + i] - ref[i]);
                    if (!(e <= 2e-5 + 1e-4 * std::fabs((double)ref[i]))) ok = false;
                    if (e > worst || std::isnan(e)) worst = e;
                }
            }
        check(ok, "paged Q8_0 layer steps (4 layers x 6 sequences) vs oracle", step, worst);
        for (int& p : pos) p++;
    }
    bool pools_ok = true;
    std::vector<uint8_t> hp(pool_b);
    for (int l = 0; l < L; l++) {
        ABI(tmac_memcpy_d2h(t, s, hp.data(), kp[l], pool_b));
        ABI(tmac_stream_synchronize(t, s));
        pools_ok &= hp == scatter(dk, l);
        ABI(tmac_memcpy_d2h(t, s, hp.data(), vp[l], pool_b));
        ABI(tmac_stream_synchronize(t, s));
        pools_ok &= hp == scatter(dv, l);
    }
    check(pools_ok, "K/V page pools byte-identical to the oracle's rows", steps, 0);
    check(tmac_check_device_error(t) == 0, "device error word clear", steps, 0);

    ABI(tmac_graph_destroy(t, g));
    for (int l = 0; l < L; l++) {
        tmac_free(t, kp[l]);
        tmac_free(t, vp[l]);
    }
    for (void* p : {(void*)d_table, (void*)d_pos, (void*)d_q, (void*)d_kn, (void*)d_vn, (void*)d_out}) tmac_free(t, p);
    tmac_stream_destroy(t, s);
    tmac_shutdown(t);
    std::printf("%s (%d failures)\n", failures ? "FAIL" : "ALL PASS", failures);
    return failures ? 1 : 0;
}
