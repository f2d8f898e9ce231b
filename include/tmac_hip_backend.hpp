// tmac_hip_backend.hpp -- C++ mirror of the reference engine's backend
// interface for the attention path, over the C ABI of tmac_attn.h.
//
// The reference engine (tmac_gguf.cpp) drives its GPU through
// namespace metal_backend (metal_backend.hpp).  For the attention slice of its
// per-layer loop (tmac_gguf.cpp:1562-1568) it calls:
//
//   metal_backend::init(ctx)                         metal_backend.cpp:21-89
//   metal_backend::metal_batch_begin(ctx)            metal_backend.hpp:114-122
//   metal_backend::rope_op(ctx, data, n_heads, head_dim, pos, base)      :381-396
//   metal_backend::elem_op(ctx, 2, cache_row, src, dim)                  :354-379
//   metal_backend::fused_qkv_op(ctx, Wq, Wk, Wv, x, q, k, v, ...)       :456-489
//   metal_backend::elem_op(ctx, 0, q|k|v, bias, dim)  (bias adds, tmac_gguf.cpp:1484-1489)
//   metal_backend::matmul_q5_0 / matmul_q8_0(ctx, rows, cols, W, x, y)   :320-338
//   metal_backend::matmul_q4_k / matmul_q6_k(ctx, rows, cols, W, x, y)   :340-350
//   metal_backend::elem_op(ctx, 0, hidden, attn_out, dim)  (residual, tmac_gguf.cpp:1499)
//   metal_backend::attention_op(ctx, Q, K, V, out, n_head, n_kv_head, head_dim, past_len) :413-453
//   metal_backend::metal_batch_end()                 metal_backend.hpp:176-190
//   metal_backend::shutdown(ctx)                     metal_backend.hpp:520
//
// hip_backend keeps those names, argument meanings and error behaviour:
// dispatch calls return void and only record work; init returns false (and
// prints a tagged message) on failure; batch_end runs the recorded step and
// waits for it.  Differences, all forced by the device model: buffers are
// device pointers (the reference wraps unified host memory), batch_begin/end
// take the context explicitly (the reference keeps it global), and the first
// failing status of a step is kept in Context::last_status instead of being
// dropped.  The recorded step is a hipGraph: the first batch instantiates it,
// later batches update it in place (hipGraphExecUpdate) when the topology is
// unchanged, so a decode step costs one graph launch.
#pragma once

#include <cstdio>

#include "tmac_attn.h"

namespace hip_backend {

struct Context {
    tmac_context* ctx = nullptr;
    tmac_stream stream = nullptr;
    tmac_graph* step = nullptr;  // executable graph of the last recorded batch
    bool recording = false;
    bool initialized = false;
    int last_status = TMAC_OK;   // first failure since batch_begin (TMAC_OK if none)
};

namespace detail {
inline void note(Context& c, int rc, const char* what) {
    if (rc == TMAC_OK) return;
    if (c.last_status == TMAC_OK) c.last_status = rc;
    std::printf("[HIP] %s: %s (%s)\n", what, tmac_status_string(rc), tmac_last_error(c.ctx));
}
}  // namespace detail

// metal_backend::init.  `rope_base`/`max_seq` size the RoPE table up front so
// that rope_op can be recorded into a step (tables cannot grow during capture).
inline bool init(Context& c, int device = 0, float rope_base = 1000000.0f, int max_seq = 256) {
    int rc = tmac_init(&c.ctx, device);
    if (rc != TMAC_OK) {
        std::printf("[HIP] init on device %d failed: %s\n", device, tmac_status_string(rc));
        return false;
    }
    if ((rc = tmac_stream_create(c.ctx, &c.stream)) != TMAC_OK ||
        (rc = tmac_rope_prepare(c.ctx, 64, rope_base, max_seq)) != TMAC_OK) {
        std::printf("[HIP] init: %s (%s)\n", tmac_status_string(rc), tmac_last_error(c.ctx));
        tmac_shutdown(c.ctx);
        c.ctx = nullptr;
        return false;
    }
    c.initialized = true;
    return true;
}

inline void shutdown(Context& c) {
    if (!c.ctx) return;
    if (c.step) tmac_graph_destroy(c.ctx, c.step);
    if (c.stream) tmac_stream_destroy(c.ctx, c.stream);
    tmac_shutdown(c.ctx);
    c = Context{};
}

// metal_batch_begin: start recording one step.
inline void batch_begin(Context& c) {
    c.last_status = TMAC_OK;
    int rc = tmac_step_begin(c.ctx, c.stream);
    c.recording = (rc == TMAC_OK);
    detail::note(c, rc, "batch_begin");
}

// metal_batch_end: finish recording, run the step and wait for it.
inline void batch_end(Context& c) {
    if (!c.recording) return;
    c.recording = false;
    int rc = tmac_step_end(c.ctx, c.stream, &c.step);
    detail::note(c, rc, "batch_end");
    if (rc != TMAC_OK || c.last_status != TMAC_OK) return;
    detail::note(c, tmac_graph_launch(c.ctx, c.step, c.stream), "batch_end: launch");
    detail::note(c, tmac_stream_synchronize(c.ctx, c.stream), "batch_end: wait");
}

inline void attention_op(Context& c, const float* Q, const float* K_cache, const float* V_cache, float* output,
                         int n_head, int n_kv_head, int head_dim, int past_len) {
    detail::note(c, tmac_attention_op(c.ctx, c.stream, Q, K_cache, V_cache, output, n_head, n_kv_head, head_dim,
                                      past_len),
                 "attention_op");
}

inline void rope_op(Context& c, float* data, int n_heads, int head_dim, int pos, float base) {
    detail::note(c, tmac_rope_op(c.ctx, c.stream, data, n_heads, head_dim, pos, base), "rope_op");
}

inline void elem_op(Context& c, int op, float* data, const float* aux, int dim) {
    detail::note(c, tmac_elem_op(c.ctx, c.stream, op, data, aux, dim), "elem_op");
}

inline void fused_qkv_op(Context& c, const uint8_t* W_q, const uint8_t* W_k, const uint8_t* W_v, const float* x,
                         float* y_q, float* y_k, float* y_v, int q_rows, int k_rows, int v_rows, int cols,
                         bool v_is_q8) {
    detail::note(c, tmac_fused_qkv_op(c.ctx, c.stream, W_q, W_k, W_v, x, y_q, y_k, y_v, q_rows, k_rows, v_rows,
                                      cols, v_is_q8 ? 1 : 0),
                 "fused_qkv_op");
}

// fused_qkv_op followed by the three bias adds, in one launch (null bias = absent).
inline void fused_qkv_bias_op(Context& c, const uint8_t* W_q, const uint8_t* W_k, const uint8_t* W_v,
                              const float* x, const float* b_q, const float* b_k, const float* b_v, float* y_q,
                              float* y_k, float* y_v, int q_rows, int k_rows, int v_rows, int cols, bool v_is_q8) {
    detail::note(c, tmac_fused_qkv_bias(c.ctx, c.stream, W_q, W_k, W_v, x, b_q, b_k, b_v, y_q, y_k, y_v, q_rows,
                                        k_rows, v_rows, cols, v_is_q8 ? 1 : 0),
                 "fused_qkv_bias_op");
}

inline void matmul_q8_0(Context& c, int rows, int cols, const uint8_t* w, const float* x, float* y) {
    detail::note(c, tmac_matmul_q8_0(c.ctx, c.stream, rows, cols, w, x, y), "matmul_q8_0");
}

inline void matmul_q5_0(Context& c, int rows, int cols, const uint8_t* w, const float* x, float* y) {
    detail::note(c, tmac_matmul_q5_0(c.ctx, c.stream, rows, cols, w, x, y), "matmul_q5_0");
}

inline void matmul_q4_k(Context& c, int rows, int cols, const uint8_t* w, const float* x, float* y) {
    detail::note(c, tmac_matmul_q4_k(c.ctx, c.stream, rows, cols, w, x, y), "matmul_q4_k");
}

inline void matmul_q6_k(Context& c, int rows, int cols, const uint8_t* w, const float* x, float* y) {
    detail::note(c, tmac_matmul_q6_k(c.ctx, c.stream, rows, cols, w, x, y), "matmul_q6_k");
}

// y += W x: the output projection and the residual add in one launch.
inline void matmul_add_op(Context& c, int qtype, int rows, int cols, const uint8_t* w, const float* x, float* y) {
    detail::note(c, tmac_matmul_add(c.ctx, c.stream, qtype, rows, cols, w, x, y), "matmul_add_op");
}

// One launch for the whole slice rope q, rope k, write k, write v, attention.
inline void layer_attention_op(Context& c, const float* q, const float* k_new, const float* v_new,
                               float* k_cache_layer, float* v_cache_layer, float* output, int n_head,
                               int n_kv_head, int head_dim, int pos, int capacity, float base) {
    detail::note(c, tmac_layer_attention(c.ctx, c.stream, q, k_new, v_new, k_cache_layer, v_cache_layer, output,
                                         n_head, n_kv_head, head_dim, pos, capacity, base),
                 "layer_attention_op");
}

}  // namespace hip_backend
