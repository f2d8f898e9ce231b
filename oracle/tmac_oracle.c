/*
 * tmac_oracle.c -- CPU restatement of the reference's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and CPU baseline for
 * libtmac_attn.so.  Nothing in the product links or calls it.
 *
 * Each function cites the reference lines it follows (liuwantao3/tmac_gguf.cpp).
 * Parity build: gcc -O2 -ffp-contract=off (no fused multiply-add, glibc libm).
 */
#include "tmac_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* RNG.  splitmix64 (Steele, Lea, Flood 2014) seeds xoshiro256** (Blackman,  */
/* Vigna 2018); normals by the Box-Muller transform in double, cast to fp32. */
/* ------------------------------------------------------------------------ */
uint64_t tmac_splitmix64(uint64_t* state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

void tmac_rng_seed(tmac_rng* r, uint64_t seed) {
    uint64_t st = seed;
    for (int i = 0; i < 4; i++) r->s[i] = tmac_splitmix64(&st);
    r->has_spare = 0;
    r->spare = 0.0;
}

void tmac_rng_set_state(tmac_rng* r, const uint64_t state[4]) {
    for (int i = 0; i < 4; i++) r->s[i] = state[i];
    r->has_spare = 0;
    r->spare = 0.0;
}

uint64_t tmac_rng_next(tmac_rng* r) {
    uint64_t* s = r->s;
    const uint64_t result = rotl64(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}

double tmac_rng_uniform(tmac_rng* r) { return (double)(tmac_rng_next(r) >> 11) * 0x1.0p-53; }

void tmac_rng_normal_f32(tmac_rng* r, float* out, size_t n) {
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i++) {
        if (r->has_spare) {
            r->has_spare = 0;
            out[i] = (float)r->spare;
            continue;
        }
        double u1 = 1.0 - tmac_rng_uniform(r); /* (0, 1] so log() is finite */
        double u2 = tmac_rng_uniform(r);
        double rad = sqrt(-2.0 * log(u1));
        double a = two_pi * u2;
        r->spare = rad * sin(a);
        r->has_spare = 1;
        out[i] = (float)(rad * cos(a));
    }
}

void tmac_fill_normal(uint64_t seed, float* out, size_t n) {
    tmac_rng r;
    tmac_rng_seed(&r, seed);
    tmac_rng_normal_f32(&r, out, n);
}

/* ------------------------------------------------------------------------ */
/* RoPE -- tmac_gguf.cpp:990-1016.  GPT-J style: adjacent pairs (d, d+1),    */
/* theta = 1/powf(base, d/head_dim) for even d, angle = pos*theta in fp32.   */
/* ------------------------------------------------------------------------ */
void oracle_rope_heads(float* x, int n_heads, int head_dim, int pos, float base) {
    for (int h = 0; h < n_heads; h++) {                                /* :992 / :1004 */
        for (int d = 0; d < head_dim; d += 2) {                        /* :993 / :1005 */
            float theta = 1.0f / powf(base, (float)d / head_dim);      /* :994 */
            float freq = pos * theta;                                  /* :995 */
            float cos_val = cosf(freq);                                /* :996 */
            float sin_val = sinf(freq);                                /* :997 */
            int idx = h * head_dim + d;                                /* :998 */
            float x0 = x[idx], x1 = x[idx + 1];                        /* :999 */
            x[idx] = x0 * cos_val - x1 * sin_val;                      /* :1000 */
            x[idx + 1] = x0 * sin_val + x1 * cos_val;                  /* :1001 */
        }
    }
}

void oracle_rope(float* q, float* k, int n_head, int n_kv_head, int head_dim, int pos, float base) {
    oracle_rope_heads(q, n_head, head_dim, pos, base);    /* :992-1003 */
    oracle_rope_heads(k, n_kv_head, head_dim, pos, base); /* :1004-1015 */
}

void oracle_rope_theta(float* theta, int head_dim, float base) {
    for (int d = 0; d < head_dim; d += 2) theta[d / 2] = 1.0f / powf(base, (float)d / head_dim);
}

/* ------------------------------------------------------------------------ */
/* Cache write -- tmac_gguf.cpp:1090-1091.                                   */
/* ------------------------------------------------------------------------ */
void oracle_cache_write(float* cache_row, const float* src, int dim) {
    for (int i = 0; i < dim; i++) cache_row[i] = src[i];
}

/* ------------------------------------------------------------------------ */
/* Attention -- tmac_gguf.cpp:1093-1128, one query head.                    */
/* `scores` has room for past_len+1 floats.                                  */
/* ------------------------------------------------------------------------ */
static void attention_head(const float* qh_data, const float* k_cache, const float* v_cache,
                           float* ctx_h, float* scores, int kv, int n_kv_head, int head_dim,
                           int past_len) {
    const int pos = past_len;
    const size_t row = (size_t)n_kv_head * head_dim; /* K_DIM: one cache row per position */

    for (int d = 0; d < head_dim; d++) ctx_h[d] = 0.0f;                       /* :1094 memset */
    for (int p = 0; p <= pos; p++) scores[p] = 0;                             /* :1104 */
    for (int d = 0; d < head_dim; d++) {                                      /* :1105 */
        float q_val = qh_data[d];                                             /* :1106 */
        for (int p = 0; p <= pos; p++) {                                      /* :1107 */
            const float* k_cached = k_cache + (size_t)p * row + (size_t)kv * head_dim; /* :1108 */
            scores[p] += q_val * k_cached[d];                                 /* :1109 */
        }
    }
    for (int p = 0; p <= pos; p++) scores[p] /= sqrtf((float)head_dim);      /* :1112 */

    float max_score = scores[0];                                              /* :1114 */
    for (int p = 1; p <= pos; p++)
        if (scores[p] > max_score) max_score = scores[p];                     /* :1115 */
    float exp_sum = 0;                                                        /* :1116 */
    for (int p = 0; p <= pos; p++) exp_sum += expf(scores[p] - max_score);    /* :1117 */
    float log_sum = logf(exp_sum) + max_score;                                /* :1118 */

    for (int p = 0; p <= pos; p++) {                                          /* :1120 */
        const float* v_cached = v_cache + (size_t)p * row + (size_t)kv * head_dim; /* :1121 */
        float exp_score = expf(scores[p] - log_sum);                          /* :1122 */
        for (int d = 0; d < head_dim; d++) ctx_h[d] += exp_score * v_cached[d]; /* :1123-1124 */
    }
}

static int bad_shape(int n_head, int n_kv_head, int head_dim, int past_len) {
    return n_head <= 0 || n_kv_head <= 0 || head_dim <= 0 || past_len < 0 ||
           (n_head % n_kv_head) != 0;
}

int oracle_attention(const float* q, const float* k_cache, const float* v_cache, float* out,
                     int n_head, int n_kv_head, int head_dim, int past_len) {
    if (bad_shape(n_head, n_kv_head, head_dim, past_len)) return -1;
    float* scores = (float*)malloc(sizeof(float) * ((size_t)past_len + 1));
    if (!scores) return -1;
    int q_per_kv = n_head / n_kv_head;                                        /* :1096 */
    for (int qh = 0; qh < n_head; qh++) {                                     /* :1098 */
        int kv = qh / q_per_kv;                                               /* :1099 */
        attention_head(q + (size_t)qh * head_dim, k_cache, v_cache, out + (size_t)qh * head_dim,
                       scores, kv, n_kv_head, head_dim, past_len);
    }
    free(scores);
    return 0;
}

int oracle_layer_step(float* q, float* k_new, const float* v_new,
                      float* k_cache_layer, float* v_cache_layer, float* out,
                      int n_head, int n_kv_head, int head_dim, int pos, float base) {
    if (bad_shape(n_head, n_kv_head, head_dim, pos)) return -1;
    const int kdim = n_kv_head * head_dim;
    oracle_rope(q, k_new, n_head, n_kv_head, head_dim, pos, base);               /* :1085-1088 */
    oracle_cache_write(k_cache_layer + (size_t)pos * kdim, k_new, kdim);         /* :1090 */
    oracle_cache_write(v_cache_layer + (size_t)pos * kdim, v_new, kdim);         /* :1091 */
    return oracle_attention(q, k_cache_layer, v_cache_layer, out,                /* :1093-1128 */
                            n_head, n_kv_head, head_dim, pos);
}

/* One decode step of the attention slice over n_layers layers, as the
 * reference's per-layer loop runs it (tmac_gguf.cpp:1537-1568 around
 * forward_layer_with_cache): layer l takes q + l*n_head*hd, k_new / v_new +
 * l*kdim, its cache at + l*capacity*kdim, and writes out + l*n_head*hd.
 * q and k_new are rotated in place. */
int oracle_decode_step(float* q, float* k_new, const float* v_new, float* k_cache, float* v_cache,
                       float* out, int n_layers, int capacity, int n_head, int n_kv_head, int head_dim,
                       int pos, float base) {
    if (n_layers < 1 || capacity < 1 || pos >= capacity) return -1;
    const size_t qd = (size_t)n_head * head_dim, kdim = (size_t)n_kv_head * head_dim;
    for (int l = 0; l < n_layers; l++) {
        const int rc = oracle_layer_step(q + l * qd, k_new + l * kdim, v_new + l * kdim,
                                         k_cache + (size_t)l * capacity * kdim,
                                         v_cache + (size_t)l * capacity * kdim, out + l * qd, n_head,
                                         n_kv_head, head_dim, pos, base);
        if (rc) return rc;
    }
    return 0;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Runs the per-head computation for every (unit, head); `units` rows each name
 * a q row, a cache base and a past_len. */
typedef struct {
    const float* q;
    const float* k;
    const float* v;
    float* out;
    int past_len;
} unit_desc;

static int run_units(const unit_desc* units, long n_units, int n_head, int n_kv_head,
                     int head_dim, int n_threads) {
    int max_past = 0;
    for (long u = 0; u < n_units; u++) {
        if (bad_shape(n_head, n_kv_head, head_dim, units[u].past_len)) return -1;
        if (units[u].past_len > max_past) max_past = units[u].past_len;
    }
    const int q_per_kv = n_head / n_kv_head;
    const long n_work = n_units * n_head;
    int rc = 0;
#ifdef _OPENMP
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads)
#endif
    {
        float* scores = (float*)malloc(sizeof(float) * ((size_t)max_past + 1));
        if (!scores) {
#ifdef _OPENMP
#pragma omp atomic write
#endif
            rc = -1;
        } else {
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
            for (long w = 0; w < n_work; w++) {
                const unit_desc* ud = &units[w / n_head];
                int qh = (int)(w % n_head);
                attention_head(ud->q + (size_t)qh * head_dim, ud->k, ud->v,
                               ud->out + (size_t)qh * head_dim, scores, qh / q_per_kv,
                               n_kv_head, head_dim, ud->past_len);
            }
            free(scores);
        }
    }
    (void)n_threads;
    return rc;
}

int oracle_attention_ragged(const float* q, const float* k_pool, const float* v_pool,
                            const int64_t* offsets, const int32_t* lengths, float* out,
                            int n_seq, int n_head, int n_kv_head, int head_dim, int n_threads) {
    if (n_seq < 0) return -1;
    if (n_seq == 0) return 0;
    unit_desc* units = (unit_desc*)malloc(sizeof(unit_desc) * (size_t)n_seq);
    if (!units) return -1;
    const size_t row = (size_t)n_kv_head * head_dim;
    const size_t qsz = (size_t)n_head * head_dim;
    for (int s = 0; s < n_seq; s++) {
        if (lengths[s] < 1 || offsets[s] < 0) { free(units); return -1; }
        units[s].q = q + (size_t)s * qsz;
        units[s].k = k_pool + (size_t)offsets[s] * row;
        units[s].v = v_pool + (size_t)offsets[s] * row;
        units[s].out = out + (size_t)s * qsz;
        units[s].past_len = lengths[s] - 1;
    }
    int rc = run_units(units, n_seq, n_head, n_kv_head, head_dim, n_threads);
    free(units);
    return rc;
}

int oracle_prefill(const float* q, const float* k_cache, const float* v_cache, float* out,
                   int n_seq, int n_q, int prefix_len, int seq_capacity,
                   int n_head, int n_kv_head, int head_dim, int n_threads) {
    if (n_seq < 0 || n_q < 0 || prefix_len < 0 || prefix_len + n_q > seq_capacity) return -1;
    long n_units = (long)n_seq * n_q;
    if (n_units == 0) return 0;
    unit_desc* units = (unit_desc*)malloc(sizeof(unit_desc) * (size_t)n_units);
    if (!units) return -1;
    const size_t row = (size_t)n_kv_head * head_dim;
    const size_t qsz = (size_t)n_head * head_dim;
    for (int s = 0; s < n_seq; s++) {
        for (int i = 0; i < n_q; i++) {
            unit_desc* ud = &units[(long)s * n_q + i];
            ud->q = q + ((size_t)s * n_q + i) * qsz;
            ud->out = out + ((size_t)s * n_q + i) * qsz;
            ud->k = k_cache + (size_t)s * seq_capacity * row;
            ud->v = v_cache + (size_t)s * seq_capacity * row;
            ud->past_len = prefix_len + i;
        }
    }
    int rc = run_units(units, n_units, n_head, n_kv_head, head_dim, n_threads);
    free(units);
    return rc;
}

/* ---- quantized weights ---- */

/* tmac_gguf.cpp:219-231: sign * (1 + mant/1024) * 2^(exp-15), subnormals
 * mant/1024 * 2^-14, exp 31 -> inf / NaN. */
float oracle_f16_to_f32(uint16_t f16) {
    uint32_t sign = (f16 >> 15) & 0x1;
    uint32_t ex = (f16 >> 10) & 0x1F;
    uint32_t mant = f16 & 0x3FF;
    if (ex == 0) {
        if (mant == 0) return 0.0f;
        return (sign ? -1.0f : 1.0f) * (mant / 1024.0f) * powf(2.0f, -14.0f);
    }
    if (ex == 31) return mant ? NAN : (sign ? -INFINITY : INFINITY);
    return (sign ? -1.0f : 1.0f) * (1.0f + mant / 1024.0f) * powf(2.0f, (int)ex - 15);
}

/* tmac_gguf.cpp:330-366: element (half, sub, l) of a 210-byte super-block:
 * 4 low bits from ql (sub 0/2: bytes l, sub 1/3: bytes l + 32, low nibble for
 * sub 0/1, high for 2/3), 2 high bits from qh byte l at shift 2*sub, minus 32;
 * times the int8 scale l / 16 + 2*sub and d, multiplied in that order. */
static float dequant_q6_k(const uint8_t* data, uint64_t idx) {
    const uint64_t block = idx / 256, offset = idx % 256, base = block * 210;
    const float d = oracle_f16_to_f32((uint16_t)(data[base + 208] | (data[base + 209] << 8)));
    const uint64_t half = offset / 128, pos = offset % 128, l = pos % 32, sub = pos / 32;
    const uint64_t ql_base = base + half * 64, qh_base = base + 128 + half * 32, sc_base = base + 192 + half * 8;
    const uint8_t ql_byte = data[ql_base + l + ((sub & 1) ? 32 : 0)];
    const uint8_t ql = (sub < 2) ? (ql_byte & 0xF) : (ql_byte >> 4);
    const uint8_t qh = (data[qh_base + l] >> (2 * sub)) & 0x3;
    const int8_t q = (int8_t)((qh << 4) | ql) - 32;
    const int8_t scale = (int8_t)data[sc_base + l / 16 + sub * 2];
    return d * scale * q;
}

/* tmac_gguf.cpp:368-397: sub-block sb = e / 32 of a 144-byte super-block;
 * nibble of qs[(sb / 2) * 32 + e % 32] (low for even sb); 6-bit scale and min
 * unpacked from the 12 scale bytes; w = d * sc * q - dmin * m. */
static float dequant_q4_k(const uint8_t* data, uint64_t idx) {
    const uint64_t block = idx / 256, offset = idx % 256, base = block * 144;
    const float d = oracle_f16_to_f32((uint16_t)(data[base] | (data[base + 1] << 8)));
    const float dmin = oracle_f16_to_f32((uint16_t)(data[base + 2] | (data[base + 3] << 8)));
    const uint64_t sb = offset / 32, q_pos = offset % 32;
    const uint8_t qs_byte = data[base + 16 + (sb / 2) * 32 + q_pos];
    const uint8_t q4 = (sb % 2 == 0) ? (qs_byte & 0xF) : (qs_byte >> 4);
    const uint8_t* sc6 = data + base + 4;
    uint8_t sc, m;
    if (sb < 4) {
        sc = sc6[sb] & 63;
        m = sc6[sb + 4] & 63;
    } else {
        sc = (sc6[sb + 4] & 0xF) | ((sc6[sb - 4] >> 6) << 4);
        m = (sc6[sb + 4] >> 4) | ((sc6[sb] >> 6) << 4);
    }
    return d * (float)sc * (float)q4 - dmin * (float)m;
}

/* tmac_gguf.cpp:240-250 (Q8_0), 311-327 (Q5_0), 330-397 (Q6_K, Q4_K): the weight at flat index idx. */
float oracle_dequant(int type, const uint8_t* data, uint64_t idx) {
    if (type == ORACLE_Q6_K) return dequant_q6_k(data, idx);
    if (type == ORACLE_Q4_K) return dequant_q4_k(data, idx);
    const uint64_t block = idx / 32, e = idx % 32;
    if (type == ORACLE_Q8_0) {
        const uint8_t* b = data + block * 34;
        const float d = oracle_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
        return (float)(int8_t)b[2 + e] * d;
    }
    const uint8_t* b = data + block * 22;
    const float d = oracle_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
    const uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
    const uint8_t byte = b[6 + (e < 16 ? e : e - 16)];
    const uint8_t ql = e < 16 ? (byte & 0xF) : (byte >> 4);
    const int q = (int)((((qh >> e) & 1) << 4) | ql) - 16;
    return d * (float)q;
}

/* tmac_gguf.cpp:510-514: one fp32 accumulator per row, inputs in ascending
 * order, the product rounded before the add (no contraction in this build).
 * read_tensor's flat index is col + row * cols (tmac_gguf.cpp:405). */
int oracle_matmul_q(int type, const uint8_t* w, const float* x, float* y, int rows, int cols) {
    const int kquant = (type == ORACLE_Q4_K || type == ORACLE_Q6_K);
    if (!w || !x || !y || rows < 0 || cols <= 0 || cols % (kquant ? 256 : 32) ||
        (type != ORACLE_Q5_0 && type != ORACLE_Q8_0 && !kquant))
        return -1;
    for (int i = 0; i < rows; i++) {
        float sum = 0;
        for (int j = 0; j < cols; j++) sum += oracle_dequant(type, w, (uint64_t)j + (uint64_t)i * cols) * x[j];
        y[i] = sum;
    }
    return 0;
}

/* tmac_gguf.cpp:1046-1081: the three projections of the normed hidden state,
 * then `out[i] += b[i]` for each bias that exists. */
int oracle_qkv(const uint8_t* wq, const uint8_t* wk, const uint8_t* wv, int v_is_q8, const float* x,
               const float* bq, const float* bk, const float* bv, float* q, float* k, float* v,
               int q_rows, int k_rows, int v_rows, int cols) {
    if (oracle_matmul_q(ORACLE_Q5_0, wq, x, q, q_rows, cols) ||
        oracle_matmul_q(ORACLE_Q5_0, wk, x, k, k_rows, cols) ||
        oracle_matmul_q(v_is_q8 ? ORACLE_Q8_0 : ORACLE_Q5_0, wv, x, v, v_rows, cols))
        return -1;
    if (bq) for (int i = 0; i < q_rows; i++) q[i] += bq[i];
    if (bk) for (int i = 0; i < k_rows; i++) k[i] += bk[i];
    if (bv) for (int i = 0; i < v_rows; i++) v[i] += bv[i];
    return 0;
}

/* ---- Q8_0 requantization ---- */

/* scripts/extract_tmac.py:53-74, bit for bit. */
uint16_t oracle_f32_to_f16_trunc(float v) {
    uint32_t bits;
    memcpy(&bits, &v, 4);
    if (v == 0.0f) return 0;
    const uint32_t sign = (bits >> 31) & 1, ex = (bits >> 23) & 0xFF, mant = bits & 0x7FFFFF;
    if (ex == 0) return 0;
    uint32_t ex16, mant16;
    if (ex >= 0x8F) {
        ex16 = 31;
        mant16 = 0;
    } else if (ex <= 0x70) {
        ex16 = 0;
        mant16 = 0;
    } else {
        ex16 = ex - 127 + 15;
        mant16 = mant >> 13;
    }
    return (uint16_t)((sign << 15) | (ex16 << 10) | mant16);
}

/* scripts/extract_tmac.py:159-173.  numpy evaluates max_abs / 127.0 and
 * fp32_block / d either entirely in float32 (numpy >= 2) or as a float64
 * quotient that is rounded to float32 before use (numpy 1.x value-based
 * casting); both give the correctly rounded float32 quotient, which is what
 * the float divisions below compute.  np.round rounds half to even: rintf in
 * the default rounding mode. */
void oracle_quantize_q8_0_block(const float* x, uint8_t* block) {
    float max_abs = 0.0f;
    for (int i = 0; i < 32; i++) {
        const float a = fabsf(x[i]);
        if (a > max_abs) max_abs = a;
    }
    const float d = ((double)max_abs < 1e-10) ? 1.0f : max_abs / 127.0f;
    const uint16_t d_bits = oracle_f32_to_f16_trunc(d);
    block[0] = (uint8_t)(d_bits & 0xFF);
    block[1] = (uint8_t)(d_bits >> 8);
    for (int i = 0; i < 32; i++) {
        const float q = rintf(x[i] / d);
        block[2 + i] = (uint8_t)(int8_t)(int)q;
    }
}

void oracle_q8_kv_rows(const float* x, int64_t n_head_rows, uint8_t* out) {
    uint8_t blk[34];
    for (int64_t r = 0; r < n_head_rows; r++) {
        uint8_t* o = out + r * 68;
        for (int b = 0; b < 2; b++) {
            oracle_quantize_q8_0_block(x + r * 64 + 32 * b, blk);
            memcpy(o + 32 * b, blk + 2, 32);
            o[64 + 2 * b] = blk[0];
            o[65 + 2 * b] = blk[1];
        }
    }
}

void oracle_q8_kv_widen(const uint8_t* rows, int64_t n_head_rows, float* out) {
    for (int64_t r = 0; r < n_head_rows; r++) {
        const uint8_t* o = rows + r * 68;
        for (int e = 0; e < 64; e++) {
            const int b = e / 32;
            const float scale = oracle_f16_to_f32((uint16_t)(o[64 + 2 * b] | (o[65 + 2 * b] << 8)));
            const int8_t val = (int8_t)o[e];
            out[r * 64 + e] = val * scale;
        }
    }
}
