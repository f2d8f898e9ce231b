/*
 * tmac_oracle.h -- CPU restatement of the reference's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * implementation in libtmac_attn.so.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; no product code path calls it.
 *
 * Restated from liuwantao3/tmac_gguf.cpp (reference, read as text):
 *   RoPE          tmac_gguf.cpp:990-1016   (apply_rope)
 *   cache write   tmac_gguf.cpp:1090-1091  (g_k_cache/g_v_cache[layer][pos][i] = k_new/v_new[i])
 *   cache layout  tmac_gguf.cpp:200-201    (float [layer][pos][n_kv_head*head_dim])
 *   cache reset   tmac_gguf.cpp:1430-1434  (memset 0)
 *   attention     tmac_gguf.cpp:1093-1128  (two-pass log-sum-exp softmax)
 *   constants     tmac_gguf.cpp:163-172    (Qwen2-0.5B: 14 q heads, 2 kv heads, head_dim 64)
 *   fp16 decode   tmac_gguf.cpp:219-231    (f16_to_f32)
 *   Q8_0 / Q5_0   tmac_gguf.cpp:240-250, 311-327 (dequant_q8_0 / dequant_q5_0)
 *   Q6_K / Q4_K   tmac_gguf.cpp:330-397    (dequant_q6_k / dequant_q4_k)
 *   matmul        tmac_gguf.cpp:405-414, 510-514 (read_tensor + the CPU row loop)
 *   QKV + bias    tmac_gguf.cpp:1046-1081  (three matmuls on the normed hidden state, then bias adds)
 *   Q8_0 requant  scripts/extract_tmac.py:53-74, 159-173 (float_to_fp16, quantize_q8_0_block)
 *
 * Generalisations (the reference hard-codes them): n_head / n_kv_head /
 * head_dim / base are arguments, the score buffer is sized by n_pos instead of
 * MAX_SEQ_LEN (tmac_gguf.cpp:1103), and batched / ragged / prefill drivers loop
 * the single-sequence function.  Loop order, accumulation order and fp32 types
 * are kept statement for statement; the parity build uses -ffp-contract=off so
 * that no multiply-add is fused, as in the reference's scalar loops.
 */
#ifndef TMAC_ORACLE_H
#define TMAC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic RNG: splitmix64 seeding xoshiro256**, Box-Muller ---- */
typedef struct {
    uint64_t s[4];
    int has_spare;
    double spare;
} tmac_rng;

uint64_t tmac_splitmix64(uint64_t* state);
void tmac_rng_seed(tmac_rng* r, uint64_t seed);
uint64_t tmac_rng_next(tmac_rng* r);
void tmac_rng_set_state(tmac_rng* r, const uint64_t state[4]);  /* raw state (test vectors) */
double tmac_rng_uniform(tmac_rng* r);                  /* [0, 1), 53 random bits */
void tmac_rng_normal_f32(tmac_rng* r, float* out, size_t n);
/* Convenience: fill `out` with n N(0,1) floats from a fresh stream `seed`. */
void tmac_fill_normal(uint64_t seed, float* out, size_t n);

/* ---- RoPE: tmac_gguf.cpp:990-1016 ---- */
/* Rotates n_heads heads of x in place (one loop of apply_rope). */
void oracle_rope_heads(float* x, int n_heads, int head_dim, int pos, float base);
/* apply_rope(q, k, pos): q heads first, then k heads. */
void oracle_rope(float* q, float* k, int n_head, int n_kv_head, int head_dim, int pos, float base);
/* theta table for pair j (d = 2j): 1/powf(base, (float)d/head_dim), as the reference computes it. */
void oracle_rope_theta(float* theta, int head_dim, float base);

/* ---- cache write: tmac_gguf.cpp:1090-1091 ---- */
void oracle_cache_write(float* cache_row, const float* src, int dim);

/* ---- attention: tmac_gguf.cpp:1093-1128 ----
 * q   [n_head][head_dim]
 * k,v [n_pos][n_kv_head][head_dim]  (row = position, the reference layout)
 * out [n_head][head_dim]
 * Attends to positions 0..past_len inclusive.  Returns 0, or -1 on bad args. */
int oracle_attention(const float* q, const float* k_cache, const float* v_cache, float* out,
                     int n_head, int n_kv_head, int head_dim, int past_len);

/* One layer of the reference decode step restricted to the hot path
 * (tmac_gguf.cpp:1085-1128): RoPE q/k in place at `pos`, write k/v to row `pos`
 * of the layer cache, then attention with past_len = pos. */
int oracle_layer_step(float* q, float* k_new, const float* v_new,
                      float* k_cache_layer, float* v_cache_layer, float* out,
                      int n_head, int n_kv_head, int head_dim, int pos, float base);

/* Batched / ragged decode: sequence s reads rows [offsets[s], offsets[s]+lengths[s])
 * of the packed k/v pools and attends to all of them (past_len = lengths[s]-1).
 * q/out are [n_seq][n_head][head_dim].  n_threads > 1 runs (seq, head) pairs on
 * OpenMP threads; each pair is computed exactly as in the serial loop. */
/* A decode step over n_layers layers (the reference's per-layer loop,
 * tmac_gguf.cpp:1537-1568): oracle_layer_step for each layer in turn; layer
 * l's cache starts l * capacity rows in. */
int oracle_decode_step(float* q, float* k_new, const float* v_new, float* k_cache, float* v_cache,
                       float* out, int n_layers, int capacity, int n_head, int n_kv_head, int head_dim,
                       int pos, float base);
int oracle_attention_ragged(const float* q, const float* k_pool, const float* v_pool,
                            const int64_t* offsets, const int32_t* lengths, float* out,
                            int n_seq, int n_head, int n_kv_head, int head_dim, int n_threads);

/* Chunked causal prefill, defined as the reference's decode applied per query
 * row (the reference has no prefill kernel; tmac_gguf.cpp:1621-1658 feeds the
 * prompt one token at a time): row i of sequence s attends to rows
 * 0..prefix_len+i of that sequence's cache.
 * q/out [n_seq][n_q][n_head][head_dim], k/v [n_seq][seq_capacity][n_kv_head][head_dim]. */
int oracle_prefill(const float* q, const float* k_cache, const float* v_cache, float* out,
                   int n_seq, int n_q, int prefix_len, int seq_capacity,
                   int n_head, int n_kv_head, int head_dim, int n_threads);

/* Number of OpenMP threads the library was built with (1 without OpenMP). */
int oracle_max_threads(void);

/* ---- quantized weights: the producer of q / k_new / v_new ----
 * Blocks of 32 weights along a row (GGML layout, rows of `cols` inputs):
 *   Q8_0 (type 8): fp16 d, int8 q[32]                          34 bytes; w = q * d
 *   Q5_0 (type 6): fp16 d, uint32 qh, uint8 qs[16]             22 bytes;
 *                  element e: low nibble of qs[e] (e < 16) or high nibble of
 *                  qs[e - 16], fifth bit = bit e of qh, w = d * (q5 - 16)     */
enum { ORACLE_Q5_0 = 6, ORACLE_Q8_0 = 8, ORACLE_Q4_K = 12, ORACLE_Q6_K = 14 };
/* Super-blocks of 256 weights (cols a multiple of 256):
 *   Q6_K (type 14): ql[128], qh[64], int8 scales[16], fp16 d              210 bytes
 *   Q4_K (type 12): fp16 d, fp16 dmin, scales[12] (6-bit sc/m), qs[128]   144 bytes  */
float oracle_f16_to_f32(uint16_t h);
float oracle_dequant(int type, const uint8_t* data, uint64_t idx);
/* y[i] = sum over j ascending of w[i][j] * x[j], one fp32 accumulator per row. */
int oracle_matmul_q(int type, const uint8_t* w, const float* x, float* y, int rows, int cols);
/* q = Wq x (+ bq), k = Wk x (+ bk), v = Wv x (+ bv); Wq, Wk are Q5_0, Wv is Q8_0
 * when v_is_q8 else Q5_0; a null bias is skipped, as the reference skips an
 * absent tensor. */
int oracle_qkv(const uint8_t* wq, const uint8_t* wk, const uint8_t* wv, int v_is_q8, const float* x,
               const float* bq, const float* bk, const float* bv, float* q, float* k, float* v,
               int q_rows, int k_rows, int v_rows, int cols);

/* ---- Q8_0 requantization (the Q8_0 KV cache) ----
 * scripts/extract_tmac.py:53-74 float_to_fp16: sign, exponent rebased
 * (exp - 127 + 15), mantissa truncated to 10 bits; 0 and fp32-subnormal
 * inputs give 0, fp32 exponents <= 0x70 give a signed zero, >= 0x8F infinity. */
uint16_t oracle_f32_to_f16_trunc(float v);
/* scripts/extract_tmac.py:159-173 quantize_q8_0_block: max_abs = max |x|,
 * d = 1 if max_abs < 1e-10 else max_abs / 127, q = round(x / d) half to even
 * (numpy), block = fp16 d (float_to_fp16) then int8 q[32]: 34 bytes. */
void oracle_quantize_q8_0_block(const float* x, uint8_t* block);
/* Q8_0 KV cache head rows (68 bytes per 64 values): the two blocks of each
 * 64 values regrouped as q[0..63], d0, d1. */
void oracle_q8_kv_rows(const float* x, int64_t n_head_rows, uint8_t* out);
/* Head rows -> fp32 with dequant_q8_0 (tmac_gguf.cpp:240-250): value = q * d. */
void oracle_q8_kv_widen(const uint8_t* rows, int64_t n_head_rows, float* out);

#ifdef __cplusplus
}
#endif
#endif
