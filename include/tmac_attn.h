/*
 * tmac_attn.h -- C ABI of the MI355X (gfx950) attention hot path of
 * liuwantao3/tmac_gguf.cpp: GQA decode attention over the fp32 KV cache,
 * RoPE, and the KV-cache row write, plus the QKV projection that feeds them.
 *
 * The reference engine calls three Metal dispatch helpers from its per-layer
 * loop (tmac_gguf.cpp:1562-1568), bracketed by metal_batch_begin/end:
 *
 *   attention_op(ctx, Q, K_cache, V_cache, output, n_head, n_kv_head, head_dim, past_len)
 *                                                    metal_backend.hpp:413-453
 *   rope_op(ctx, data, n_heads, head_dim, pos, base) metal_backend.hpp:381-396
 *   elem_op(ctx, 2, cache_row, src, dim)             metal_backend.hpp:354-379 (op 2 = copy)
 *
 * This header exports the same three operations with the same argument
 * meaning, plus context lifecycle, step capture (hipGraph, the analogue of the
 * one command buffer per decode step), a fused per-layer entry point, the
 * batched / ragged-split-KV / prefill extensions, and the producer of the
 * path's inputs: fused_qkv_op (metal_backend.hpp:456) with its bias adds.
 *
 * Conventions (all entry points):
 *  - Buffers are DEVICE pointers owned by the caller (allocate them with
 *    tmac_malloc or hipMalloc).  The library never frees caller memory.
 *  - Every call returns int status: 0 (TMAC_OK) or a TMAC_ERR_* code.  Shape
 *    and pointer checks run on the host before any launch; a rejected call
 *    launches nothing.  HIP runtime failures return TMAC_ERR_HIP_BASE + hipError_t.
 *  - Calls are stream-ordered and asynchronous; `stream` is a hipStream_t
 *    (NULL = the null stream).
 *  - A context is used from one host thread at a time, and its launches must
 *    not overlap on several streams (they share the split-KV workspace).
 *    Different contexts are independent: each may be driven from its own
 *    thread at the same time as the others (see tmac_shutdown).
 *  - Cache layout is the reference's: one row per position, row =
 *    [n_kv_head][head_dim] fp32 (tmac_gguf.cpp:200-201).
 *    Query head h reads kv head h / (n_head / n_kv_head) (tmac_gguf.cpp:1099).
 *  - Shapes.  head_dim 64 with n_head / n_kv_head = G and n_kv_head = KV in
 *    (G, KV) = (7, 2) (Qwen2-0.5B), (1, 1), (1, 2), (2, 2), (4, 2), (4, 4), (8, 1)
 *    run the compiled kernels on every entry point.  Like the reference's
 *    attention_op, which sends head_dim != 64 to kernel_attn (any group, any
 *    head_dim; metal_backend.hpp:416-452, kernel_attn.metal:7-60), the fp32
 *    entry points tmac_attention_op, tmac_attention_decode_batched /
 *    _ragged / _ragged_noalloc and tmac_layer_attention[_devpos] take any
 *    other n_head a multiple of n_kv_head and any even head_dim up to 256
 *    (one workgroup per query head; scores scaled by 1/sqrt(head_dim)), and
 *    tmac_rope_op / tmac_rope_rows any even head_dim up to 256 (kernel_rope.metal:5-22).
 *    The reference's kernel_attn is one 32-lane simdgroup with 2 dims per lane
 *    (kernel_attn.metal:20-21), so it defines head_dim <= 64 only; above 64 this
 *    library computes attention over every dimension, as the CPU restatement
 *    of tmac_gguf.cpp:1093-1128 generalised to head_dim does, with no reference
 *    result to compare against (parity there is unpinned).
 *    The bf16 / fp16 / Q8_0 caches, the paged caches and chunked prefill keep
 *    head_dim 64 and the compiled groups; other shapes return TMAC_ERR_UNSUPPORTED.
 */
#ifndef TMAC_ATTN_H
#define TMAC_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TMAC_ATTN_ABI_VERSION 1

enum tmac_status {
    TMAC_OK = 0,
    TMAC_ERR_INVALID_ARG = 1,     /* bad shape or value (negative past_len, n_head % n_kv_head, ...) */
    TMAC_ERR_NULL_POINTER = 2,
    TMAC_ERR_MISALIGNED = 3,      /* q/k/v/out/cache rows must be 16-byte aligned */
    TMAC_ERR_UNSUPPORTED = 4,     /* shape outside an entry point's domain (see Shapes), elem_op op 1 */
    TMAC_ERR_CAPACITY = 5,        /* position beyond the cache / RoPE table / workspace */
    TMAC_ERR_NOT_INITIALIZED = 6,
    TMAC_ERR_CAPTURE = 7,         /* needs an allocation while the stream is being captured, or a device-wide
                                     synchronize while a capture is in progress */
    TMAC_ERR_DEVICE_FAULT = 8,    /* a kernel reported a bad device-side position */
    TMAC_ERR_NOT_FOUND = 9,       /* no tensor of that name in a loaded weight file */
    TMAC_ERR_IO = 10,             /* weight file missing, truncated or not in TMAC format */
    TMAC_ERR_HIP_BASE = 1000      /* TMAC_ERR_HIP_BASE + hipError_t */
};

typedef struct tmac_context tmac_context;
typedef struct tmac_graph tmac_graph;
typedef void* tmac_stream;  /* hipStream_t */

/* Human-readable text for a status code (static storage). */
const char* tmac_status_string(int status);
/* Detail of the last error reported through this context (thread-unsafe, like the context). */
const char* tmac_last_error(const tmac_context* ctx);
int tmac_abi_version(void);

/* ---- lifecycle: replaces metal_backend::init / shutdown (metal_backend.cpp:21-89, .hpp:519-520) ----
 * Loads the gfx950 code object embedded in this library (hipModuleLoadData)
 * on `device`, resolves every kernel, and allocates the split-KV workspace.
 * Fails with TMAC_ERR_HIP_BASE+... when no device or no gfx950 is present. */
int tmac_init(tmac_context** ctx, int device);
/* The caller's work on the context must be finished.  Contexts are independent: several may be used
 * at the same time from different host threads (one thread per context at a time).  The library's own
 * copies and fills run on a stream of the context, and it synchronizes the whole device only while no
 * step capture of any context is in progress, so a call on one context never ends another thread's
 * capture (on this runtime a legacy-stream copy or a device-wide synchronize from any thread would). */
int tmac_shutdown(tmac_context* ctx);

/* ---- the reference's three per-layer dispatches ---- */

/* attention_op, metal_backend.hpp:413-453 / tmac_gguf.cpp:1093-1128.
 * q [n_head][64] (already rotated), k_cache/v_cache = row 0 of the layer
 * cache, out [n_head][64].  Attends rows 0..past_len inclusive. */
int tmac_attention_op(tmac_context* ctx, tmac_stream stream, const float* q, const float* k_cache,
                      const float* v_cache, float* out, int n_head, int n_kv_head, int head_dim,
                      int past_len);

/* rope_op, metal_backend.hpp:381-396 / tmac_gguf.cpp:990-1016: rotates
 * n_heads heads of `data` in place at position `pos` with frequency base
 * `base` (GPT-J adjacent pairs).  cos/sin of pos*theta come from a table the
 * context builds on the host with the platform libm (tmac_rope_prepare). */
int tmac_rope_op(tmac_context* ctx, tmac_stream stream, float* data, int n_heads, int head_dim,
                 int pos, float base);
/* rope_op over n_rows rows (row r at data + r * row_stride floats, n_heads heads each) at positions
 * first_pos + r: the RoPE of a prompt chunk before its rows are written to the cache.  Row r is
 * bit-identical to tmac_rope_op at position first_pos + r.  data and every row are 16-byte aligned
 * (row_stride a multiple of 4 floats; otherwise TMAC_ERR_MISALIGNED).  No counterpart in the reference,
 * which feeds a prompt one token at a time (tmac_gguf.cpp:1621-1658). */
int tmac_rope_rows(tmac_context* ctx, tmac_stream stream, float* data, int n_rows, int64_t row_stride, int n_heads,
                   int head_dim, int first_pos, float base);

/* elem_op, metal_backend.hpp:354-379 (kernel_elem.metal:14-21), i < dim:
 *   op 2, cache write  data[i] = aux[i]   (tmac_gguf.cpp:1090-1091, 1564-1565)
 *   op 0, add          data[i] += aux[i]  (the bias adds, tmac_gguf.cpp:1484-1489)
 * op 1 (silu * up) belongs to the FFN and returns TMAC_ERR_UNSUPPORTED. */
int tmac_elem_op(tmac_context* ctx, tmac_stream stream, int op, float* data, const float* aux, int dim);

/* ---- QKV projection, the producer of q / k_new / v_new ----
 * fused_qkv_op, metal_backend.hpp:456-489 (kernel_fused_qkv.metal:8-67); the
 * reference's CPU form is tmac_gguf.cpp:1046-1062.  y_q = W_q x, y_k = W_k x,
 * y_v = W_v x in one launch.  Each W is rows x cols in GGML blocks of 32 along
 * a row: W_q and W_k Q5_0 (22 bytes: fp16 d, u32 qh, u8 qs[16]); W_v Q8_0
 * (34 bytes: fp16 d, i8 q[32]) when v_is_q8, else Q5_0 (tmac_gguf.cpp:240-250,
 * 311-327).  cols must be a multiple of 32; x is 16-byte aligned and must not
 * overlap an output; weights are 2-byte aligned.  Each output is the exact
 * dequantised dot product rounded as an fp32 sum (the order of the sum differs
 * from the reference's sequential loop only by rounding). */
int tmac_fused_qkv_op(tmac_context* ctx, tmac_stream stream, const void* w_q, const void* w_k, const void* w_v,
                      const float* x, float* y_q, float* y_k, float* y_v, int q_rows, int k_rows, int v_rows,
                      int cols, int v_is_q8);
/* Extension: the same plus the three bias adds that follow it
 * (tmac_gguf.cpp:1484-1489, elem_op 0) in the same launch; a null bias is
 * absent, as the reference skips a missing bias tensor. */
int tmac_fused_qkv_bias(tmac_context* ctx, tmac_stream stream, const void* w_q, const void* w_k, const void* w_v,
                        const float* x, const float* b_q, const float* b_k, const float* b_v, float* y_q, float* y_k,
                        float* y_v, int q_rows, int k_rows, int v_rows, int cols, int v_is_q8);

/* ---- attention output projection, the consumer of the path's output ----
 * matmul_q8_0 / matmul_q5_0, metal_backend.hpp:320-338 (mul_mat_q5_0.metal:6-37);
 * the engine calls them through matmul() (tmac_gguf.cpp:476-490) for
 * attn_output.weight (tmac_gguf.cpp:1497-1498).  y = W x, W rows x cols in
 * Q8_0 / Q5_0 blocks as above; x 16-byte aligned, x and y disjoint. */
/* the reference's tensor type codes (tmac_gguf.cpp:176-182) */
enum tmac_weight_type { TMAC_F32 = 0, TMAC_F16 = 1, TMAC_Q5_0 = 6, TMAC_Q8_0 = 8, TMAC_Q4_K = 12, TMAC_Q6_K = 14 };
int tmac_matmul_q8_0(tmac_context* ctx, tmac_stream stream, int rows, int cols, const void* w, const float* x,
                     float* y);
int tmac_matmul_q5_0(tmac_context* ctx, tmac_stream stream, int rows, int cols, const void* w, const float* x,
                     float* y);
/* matmul_q4_k / matmul_q6_k, metal_backend.hpp:340-350: K-quant super-blocks of
 * 256 weights along a row (Q4_K 144 bytes: fp16 d, fp16 dmin, 12 bytes of
 * 6-bit scales/mins, 128 bytes of nibbles; Q6_K 210 bytes: ql[128], qh[64],
 * int8 scales[16], fp16 d; tmac_gguf.cpp:330-397).  cols a multiple of 256. */
int tmac_matmul_q4_k(tmac_context* ctx, tmac_stream stream, int rows, int cols, const void* w, const float* x,
                     float* y);
int tmac_matmul_q6_k(tmac_context* ctx, tmac_stream stream, int rows, int cols, const void* w, const float* x,
                     float* y);
/* Extension: y += W x in one launch, i.e. the projection followed by the
 * residual add elem_op(0, hidden, attn_out) (tmac_gguf.cpp:1497-1499):
 * each y[i] is (W x)[i] rounded to fp32, then added to y[i]. */
int tmac_matmul_add(tmac_context* ctx, tmac_stream stream, int qtype, int rows, int cols, const void* w,
                    const float* x, float* y);

/* ---- fused per-layer step (one launch replaces rope_op x2 + elem_op(2) x2 + attention_op,
 *      tmac_gguf.cpp:1562-1568) ----
 * Rotates q and k_new at `pos`, writes k (rotated) and v_new to row `pos` of
 * the layer cache, and attends rows 0..pos.  q/k_new/v_new are read only
 * (the rotated q is not written back).  `capacity` = rows in the layer cache. */
int tmac_layer_attention(tmac_context* ctx, tmac_stream stream, const float* q, const float* k_new,
                         const float* v_new, float* k_cache, float* v_cache, float* out, int n_head,
                         int n_kv_head, int head_dim, int pos, int capacity, float base);
/* Same, with the position read on the device from *pos_dev at run time, so a
 * captured step graph can be replayed for successive positions.  An
 * out-of-range *pos_dev makes the kernel skip its work and raise the device
 * error word (see tmac_check_device_error).
 * The context keeps a small RoPE row cache for each of the first 64 distinct
 * pos_dev counters it sees: tmac_pos_update fills it with the row of the
 * position it sets, so the step rotates q and k_new without first waiting for
 * *pos_dev.  A position written into the counter any other way is still
 * correct (the row is then read from the table after the position). */
int tmac_layer_attention_devpos(tmac_context* ctx, tmac_stream stream, const float* q,
                                const float* k_new, const float* v_new, float* k_cache,
                                float* v_cache, float* out, int n_head, int n_kv_head, int head_dim,
                                const int* pos_dev, int capacity, float base);
/* *pos_dev = value (add = 0) or *pos_dev += value (add = 1), as a kernel (graph
 * safe); for a counter the layer steps have used, also the RoPE row of the new
 * position into that counter's row cache (see tmac_layer_attention_devpos). */
int tmac_pos_update(tmac_context* ctx, tmac_stream stream, int* pos_dev, int value, int add);

/* Builds (or extends) the cos/sin table for (head_dim, base) to cover
 * positions [0, n_pos).  Synchronous; must not be called during capture.
 * rope_op / layer_attention build it on first use when not capturing. */
int tmac_rope_prepare(tmac_context* ctx, int head_dim, float base, int n_pos);

/* ---- batched decode (extensions; no counterpart in the single-sequence reference) ----
 * Sequence s reads cache rows starting at k + s*seq_stride*row (row = n_kv_head*64
 * floats) and attends its first n_pos rows; q/out are [n_seq][n_head][64]. */
int tmac_attention_decode_batched(tmac_context* ctx, tmac_stream stream, const float* q,
                                  const float* k, const float* v, float* out, int n_seq,
                                  int n_head, int n_kv_head, int head_dim, int n_pos,
                                  int64_t seq_stride);
/* Ragged split-KV decode over a packed pool: sequence s attends rows
 * [offsets[s], offsets[s] + lengths[s]) (DEVICE arrays).  max_len bounds every
 * length (it sizes the grid); a longer sequence gets a NaN output and raises
 * bit 1 of the device error word.  A sequence of length 0 produces a zero
 * output.  total_rows, if the caller knows it (sum of lengths; 0 = unknown),
 * only tunes the split length for load balance -- results do not depend on it. */
int tmac_attention_decode_ragged(tmac_context* ctx, tmac_stream stream, const float* q,
                                 const float* k_pool, const float* v_pool, const int64_t* offsets,
                                 const int32_t* lengths, float* out, int n_seq, int n_head,
                                 int n_kv_head, int head_dim, int max_len, int64_t total_rows);
/* tmac_attention_decode_ragged with no allocation: no counterpart in the reference.  For callers
 * that cannot allocate device memory (code under hipGraph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments, kernels and results; the split-KV partials go to a fixed
 * device array of TMAC_SCRATCH_BYTES that the library holds on each GPU from tmac_init until the
 * process ends, instead of the context's growable workspace, and the call never calls hipMalloc or
 * hipFree.  A call whose schedule needs more than TMAC_SCRATCH_BYTES of partials launches nothing and
 * returns TMAC_ERR_CAPACITY (at 14 query heads: stream-K batches up to about 4,000 sequences, unit-grid
 * batches up to n_seq * splits = 4,500).  Every call on one GPU shares that GPU's array (all contexts
 * and streams): calls that overlap on one GPU race.  No part of it needs to start at zero. */
#define TMAC_SCRATCH_BYTES (16u << 20)
int tmac_attention_decode_ragged_noalloc(tmac_context* ctx, tmac_stream stream, const float* q,
                                         const float* k_pool, const float* v_pool, const int64_t* offsets,
                                         const int32_t* lengths, float* out, int n_seq, int n_head,
                                         int n_kv_head, int head_dim, int max_len, int64_t total_rows);

/* ---- TMAC weight file: load_tmac (tmac_gguf.cpp:1372-1425) ----
 * The file scripts/extract_tmac.py writes (its :1-24, 261-272):
 *   "TMAC", u64 n_tensors, then per tensor u64 name_len, name bytes, u64 rows,
 *   u64 cols, u32 type (tmac_weight_type), u64 n_bytes, n_bytes of data
 * (little endian).  rows / cols are as stored: rows = outputs (ne[1]), cols =
 * inputs (ne[0]).  With a context the tensors are copied to one device
 * allocation (each at a 256-byte aligned offset); with ctx == NULL they stay in
 * host memory (inspection without a GPU).  Names of 128 bytes or more are cut
 * to their first 127, as the reference does; lookups return the first tensor
 * of a name, as get_tensor_info does.  Unlike the reference, the magic is
 * checked and there is no 512 MiB cap (TMAC_ERR_IO on a short or foreign file). */
typedef struct tmac_model tmac_model;
typedef struct {
    const char* name;  /* owned by the model */
    uint64_t rows, cols;
    uint32_t type;
    uint64_t n_bytes;
    void* data;        /* device pointer, or host pointer for a model loaded without a context */
} tmac_tensor_info;
int tmac_model_load(tmac_context* ctx, const char* path, tmac_model** model);
int tmac_model_count(const tmac_model* model);  /* number of tensors, or a negative status */
int tmac_model_tensor(const tmac_model* model, int index, tmac_tensor_info* info);
int tmac_model_find(const tmac_model* model, const char* name, tmac_tensor_info* info);  /* TMAC_ERR_NOT_FOUND */
/* Frees the model's memory; ctx must be the context it was loaded with (NULL for a host model). */
int tmac_model_free(tmac_context* ctx, tmac_model* model);

/* ---- reduced-precision KV caches (extension; the quantized cache motivated at
 *      LLAMACPP_METAL_STUDY.md:50-54) ----
 * The same cache layout with narrower elements: bf16 or fp16 (half the bytes
 * on the HBM-bound path), or Q8_0 (0.27x).  A Q8_0 cache stores each
 * (row, kv head) as a 68-byte head row: int8 q[64], then the fp16 scales d0
 * (dims 0..31) and d1 (dims 32..63), i.e. the two GGML Q8_0 blocks of those
 * 64 values (dequant_q8_0, tmac_gguf.cpp:240-250: value = q * d) with the
 * scales moved behind the values; a cache row is n_kv_head * 68 bytes.
 * Rows are read and widened exactly to fp32, so each call equals the fp32
 * path run on the widened cache (the tolerance contract:
 * |out - oracle(widen(cache))| <= 2e-5 + 1e-4 |ref|).  The layer step turns
 * the rotated k and v_new into the cache type before it stores and attends
 * them: bf16/fp16 round to nearest even; Q8_0 quantizes each 32-value block
 * as the reference's quantize_q8_0_block does (scripts/extract_tmac.py:159-173:
 * d = max|x| / 127, or 1 when max|x| < 1e-10; q = x / d rounded half to even;
 * d stored with float_to_fp16, :53-74, which truncates the mantissa and
 * flushes fp16-subnormal values to 0).  These calls use the default 8-wave
 * group and head kernels whatever TMAC_OPT_GROUP_WAVES / _HEAD_WAVES say. */
enum tmac_kv_dtype { TMAC_KV_F32 = 0, TMAC_KV_BF16 = 1, TMAC_KV_F16 = 2, TMAC_KV_Q8_0 = 3 };
int tmac_attention_decode_batched_kv(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                                     const void* k, const void* v, float* out, int n_seq, int n_head,
                                     int n_kv_head, int head_dim, int n_pos, int64_t seq_stride);
int tmac_attention_decode_ragged_kv(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                                    const void* k_pool, const void* v_pool, const int64_t* offsets,
                                    const int32_t* lengths, float* out, int n_seq, int n_head, int n_kv_head,
                                    int head_dim, int max_len, int64_t total_rows);
int tmac_layer_attention_kv(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                            const float* k_new, const float* v_new, void* k_cache, void* v_cache, float* out,
                            int n_head, int n_kv_head, int head_dim, int pos, int capacity, float base);
int tmac_layer_attention_devpos_kv(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                                   const float* k_new, const float* v_new, void* k_cache, void* v_cache,
                                   float* out, int n_head, int n_kv_head, int head_dim, const int* pos_dev,
                                   int capacity, float base);
/* Fills a narrow cache from n fp32 values: BF16 / F16 dst[i] = src[i] rounded to nearest even;
 * Q8_0 (n % 64 == 0, src 16-byte aligned) n / 64 head rows quantized as the layer step does. */
int tmac_kv_convert(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* src, void* dst, int64_t n);

/* ---- paged KV caches (extension; the 16-token pages planned at
 *      LLAMACPP_METAL_STUDY.md:97-101, 155-162) ----
 * K and V are pools of n_pages pages of 16 rows each (a page = 16 cache rows
 * of kv_dtype, row layout as above).  block_table [n_seq][max_pages] gives,
 * for logical page j of sequence s (its rows 16j..16j+15), the pool page that
 * holds them.  An entry outside [0, n_pages) is clamped into the pool and sets
 * bit 2 of the device error word.  Pages may be shared between sequences
 * (a common prefix); the layer step must not write a row another sequence of
 * the same call reads or writes.
 *
 * Decode: sequence s attends its rows 0..lengths[s]-1 (attention_op,
 * metal_backend.hpp:354, over a paged cache); max_len >= every length and
 * max_len <= 16 * max_pages (a longer length gives NaN output and bit 1);
 * total_rows as in tmac_attention_decode_ragged.  A length of 0 gives a zero
 * output.  q/out [n_seq][n_head][64]. */
int tmac_attention_decode_paged(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                                const void* k_pages, const void* v_pages, int n_pages,
                                const int32_t* block_table, int max_pages, const int32_t* lengths,
                                float* out, int n_seq, int n_head, int n_kv_head, int head_dim,
                                int max_len, int64_t total_rows);
/* The layer step (tmac_layer_attention) for a batch of sequences on a paged
 * cache: for each s, with pos = positions[s] (device memory, so a captured step
 * replays with new positions): RoPE q[s] and k_new[s] at pos, write the rotated
 * k and v_new[s] to row pos of sequence s (tmac_gguf.cpp:1090-1091), attend
 * rows 0..pos.  q/out [n_seq][n_head][64], k_new/v_new [n_seq][n_kv_head][64].
 * max_len >= pos + 1 for every s, max_len <= 16 * max_pages; a position outside
 * [0, 16 * max_pages) sets bit 0 and skips that sequence, one in
 * [max_len, 16 * max_pages) gives NaN output and bit 1. */
int tmac_layer_attention_paged(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                               const float* k_new, const float* v_new, void* k_pages, void* v_pages,
                               int n_pages, const int32_t* block_table, int max_pages,
                               const int32_t* positions, float* out, int n_seq, int n_head, int n_kv_head,
                               int head_dim, int max_len, float base);

/* ---- chunked causal prefill (extension; the reference feeds prompts one token at a time,
 *      tmac_gguf.cpp:1621-1658, so its oracle is attention_op per query row) ----
 * Query i of sequence s sits at position prefix_len + i and attends rows
 * 0..prefix_len + i of that sequence's cache (rows prefix_len.. must already
 * hold the chunk's rotated k and v).  q/out [n_seq][n_q][n_head][64]; sequence s
 * starts at row s * seq_stride.  QK^T and PV run on bf16 MFMA (q, k, v rounded
 * to bf16, fp32 accumulation, P split into bf16 hi + lo); with bf16-exact
 * inputs the result matches the fp32 CPU path within the fp32 tolerance.
 * Two launches: the rows 0..prefix_len + n_q - 1 are first packed to bf16 tiles
 * in the context's workspace (n_seq * n_kv_head * 16 KiB per 64 rows, rounded
 * up to 256 rows), which grows on demand; a call that needs it to grow while
 * the stream is capturing returns TMAC_ERR_CAPTURE, so run the largest shape
 * once before capture. */
int tmac_attention_prefill(tmac_context* ctx, tmac_stream stream, const float* q, const float* k_cache,
                           const float* v_cache, float* out, int n_seq, int n_q, int prefix_len,
                           int64_t seq_stride, int n_head, int n_kv_head, int head_dim);
/* The same over a bf16 / fp16 / Q8_0 cache (tmac_kv_dtype; no counterpart in the
 * reference, whose cache is fp32): rows are widened exactly to fp32 and then rounded
 * to bf16 like the fp32 rows (exact for a bf16 cache). */
int tmac_attention_prefill_kv(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                              const void* k_cache, const void* v_cache, float* out, int n_seq, int n_q,
                              int prefix_len, int64_t seq_stride, int n_head, int n_kv_head, int head_dim);
/* The same over paged caches (pools of n_pages 16-row pages of kv_dtype; sequence s's row r in
 * pool page block_table[s][r / 16], as tmac_attention_decode_paged): the tile pack gathers rows
 * 0..prefix_len + n_q - 1 through the table.  prefix_len + n_q <= 16 * max_pages; an entry
 * outside the pool is clamped and sets bit 2 of the device error word. */
int tmac_attention_prefill_paged(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                                 const void* k_pages, const void* v_pages, int n_pages, const int32_t* block_table,
                                 int max_pages, float* out, int n_seq, int n_q, int prefix_len, int n_head,
                                 int n_kv_head, int head_dim);

/* Chunked prefill over a persistent bf16 tile copy of the cache (no counterpart in the
 * reference, which has no chunked prefill; for callers that prefill a prompt chunk by
 * chunk): the rows of earlier chunks are packed once, and each chunk packs only its own
 * rows before its attention.  `tiles` is a caller buffer of tmac_prefill_tiles_bytes
 * bytes for `capacity` rows per sequence (16 KiB per 64 rows and (sequence, kv head),
 * rows rounded up to 256); it is valid for the rows packed so far and the caller keeps
 * it in step with the cache (repack rows that change).
 *   tmac_prefill_pack_rows: packs rows row_begin .. row_end - 1 of every sequence, in any
 *     order and any number of times (a middle range that changed can be repacked); the
 *     other rows of the tiles keep their contents.  Cache layout and kv_dtype as
 *     tmac_attention_prefill_kv; row_end <= capacity, seq_stride >= capacity when n_seq > 1.
 *   tmac_attention_prefill_tiles: the attention of tmac_attention_prefill over the tiles,
 *     which must hold rows 0 .. prefix_len + n_q - 1 (prefix_len + n_q <= capacity).
 * pack_rows(0, prefix_len + n_q) then attention_prefill_tiles gives the outputs of
 * tmac_attention_prefill bit for bit (the same kernels on the same tiles). */
size_t tmac_prefill_tiles_bytes(int n_seq, int n_kv_head, int capacity);
int tmac_prefill_pack_rows(tmac_context* ctx, tmac_stream stream, int kv_dtype, const void* k_cache,
                           const void* v_cache, int64_t seq_stride, void* tiles, int capacity, int n_seq,
                           int n_kv_head, int head_dim, int row_begin, int row_end);
int tmac_attention_prefill_tiles(tmac_context* ctx, tmac_stream stream, const float* q, const void* tiles,
                                 int capacity, float* out, int n_seq, int n_q, int prefix_len, int n_head,
                                 int n_kv_head, int head_dim);

/* ---- tuning / introspection ---- */
enum tmac_option {
    TMAC_OPT_SPLIT_LEN = 1,     /* group kernel: rows per workgroup; 0 = automatic (default) */
    TMAC_OPT_TARGET_GROUPS = 2, /* workgroups the automatic split aims for; 0 = one per CU */
    TMAC_OPT_KERNEL = 3,        /* a tmac_kernel_choice */
    TMAC_OPT_ROTATE = 4,        /* decode: workgroup w starts w*value steps into its rows (default 0) */
    TMAC_OPT_HEAD_WAVES = 5,    /* head kernel workgroup size in waves: 4, 8 or 16 (default 8) */
    TMAC_OPT_WAVE_ORDER = 6,    /* group kernel: 0 = waves interleave steps, 1 = each wave a contiguous run */
    TMAC_OPT_GROUP_WAVES = 7,   /* fp32 group kernel workgroup size in waves: 4 or 8; 0 (default) = 4 unless a
                                   split would hold fewer than 64 rows, then 8 */
    TMAC_OPT_MFMA_DECODE = 8,   /* 1 (default): bf16/fp16/Q8_0 caches use the MFMA group kernel (decode and layer step) where one exists; 0: VALU */
    TMAC_OPT_STREAM_K = 9,      /* ragged and paged decode schedule: 1 (default) = automatic, 2 = always stream-K
                                   (the batch's rows cut into equal ranges, one workgroup each), 0 = never (one
                                   workgroup per (sequence, split) unit).  Stream-K is not used when
                                   TMAC_OPT_SPLIT_LEN is set, the head kernel is chosen or (narrow caches) the MFMA
                                   decode is off; automatic picks it, in sequences per CU, for 0.5 to 1.5 or more
                                   than 10 (fp32 ragged), from 0.5 (fp32 paged), up to 2 or more than 10 (fp32
                                   paged layer step), above 10 (bf16 / fp16 / Q8_0) */
    TMAC_OPT_HV_SPLIT = 10      /* split-V head kernel: workgroups per query head (1, 2, 4 or 8; default 8), each
                                   scoring every row and accumulating 64/value dims of V */
};
enum tmac_kernel_choice {
    TMAC_KERNEL_AUTO = 0,   /* short contexts on few sequences: the split-V head kernel (fp32 caches) or
                               the head kernel (bf16 / fp16 / Q8_0); else group */
    TMAC_KERNEL_GROUP = 1,  /* workgroup per (split, sequence), each K/V byte read once */
    TMAC_KERNEL_HEAD = 2,   /* workgroup per (query head, sequence), no split merge; 8 lanes per row */
    TMAC_KERNEL_HEADV = 3   /* the same, each query head's V dims split over TMAC_OPT_HV_SPLIT
                               workgroups (fp32 caches; other caches use the head kernel) */
};
int tmac_set_option(tmac_context* ctx, int option, int64_t value);
/* Rows per workgroup and splits the next decode with this shape would use
 * (*n_splits = 0 means the head kernel). */
int tmac_query_split(tmac_context* ctx, int n_seq, int n_pos, int n_head, int n_kv_head, int* split_len,
                     int* n_splits);
/* Reads and clears the device error word (bit 0: bad device-side position, bit 1: ragged or paged length
 * above max_len, bit 2: block-table entry outside the page pool).  Returns TMAC_ERR_DEVICE_FAULT if set.
 * Synchronizes the context's device first, unless a step capture (tmac_step_begin .. tmac_step_end) of any
 * context is in progress: a device-wide synchronize would end that capture, so the word is then read as the
 * kernels that have completed left it (synchronize the streams the work ran on before calling). */
int tmac_check_device_error(tmac_context* ctx);

/* ---- step capture: the analogue of metal_batch_begin / metal_batch_end
 *      (metal_backend.hpp:114-122, 176-190), one hipGraph per decode step ---- */
int tmac_step_begin(tmac_context* ctx, tmac_stream stream);
/* Ends capture.  *graph == NULL: instantiates a new executable graph.
 * *graph != NULL: updates it in place (hipGraphExecUpdate) and re-instantiates
 * only if the topology changed.
 * A graph keeps the addresses of the context's split-KV workspace and RoPE
 * tables that its captured launches used.  While any graph of the context is
 * alive, an eager call that needs a larger workspace or table allocates a new
 * one and keeps the old one allocated, so replays stay valid (so it does while
 * a capture of any context is in progress, when the device cannot be
 * synchronized); the kept buffers are freed when the context's last graph is
 * destroyed and no capture is in progress, or at shutdown.
 * Graphs may outlive the context (destroying one later is safe), but must not
 * be launched after tmac_shutdown. */
int tmac_step_end(tmac_context* ctx, tmac_stream stream, tmac_graph** graph);
int tmac_graph_launch(tmac_context* ctx, tmac_graph* graph, tmac_stream stream);
int tmac_graph_destroy(tmac_context* ctx, tmac_graph* graph);

/* ---- device memory, streams and events (for callers without their own HIP plumbing) ---- */
int tmac_malloc(tmac_context* ctx, void** ptr, size_t bytes);
int tmac_free(tmac_context* ctx, void* ptr);
int tmac_memcpy_h2d(tmac_context* ctx, tmac_stream stream, void* dst, const void* src, size_t bytes);
int tmac_memcpy_d2h(tmac_context* ctx, tmac_stream stream, void* dst, const void* src, size_t bytes);
int tmac_memcpy_d2d(tmac_context* ctx, tmac_stream stream, void* dst, const void* src, size_t bytes);
/* tmac_memset returns TMAC_ERR_CAPTURE on a capturing stream: a memset node in a replayed graph has not
 * reliably cleared memory on replays after the first on this GPU; clear memory before tmac_step_begin. */
int tmac_memset(tmac_context* ctx, tmac_stream stream, void* dst, int value, size_t bytes);
int tmac_stream_create(tmac_context* ctx, tmac_stream* stream);
int tmac_stream_destroy(tmac_context* ctx, tmac_stream stream);
int tmac_stream_synchronize(tmac_context* ctx, tmac_stream stream);
/* TMAC_ERR_CAPTURE while a step capture of any context is in progress (a device-wide synchronize
 * would end it): synchronize the streams instead. */
int tmac_device_synchronize(tmac_context* ctx);
typedef void* tmac_event;   /* hipEvent_t */
int tmac_event_create(tmac_context* ctx, tmac_event* ev);
int tmac_event_destroy(tmac_context* ctx, tmac_event ev);
int tmac_event_record(tmac_context* ctx, tmac_event ev, tmac_stream stream);
int tmac_event_elapsed_ms(tmac_context* ctx, tmac_event start, tmac_event stop, float* ms);
/* Device facts: compute units, HBM bus width etc. are in the returned text. */
int tmac_device_info(tmac_context* ctx, char* buf, size_t buf_len, int* n_cu);

/* ---- synthetic workload streams (host only; no counterpart in the reference, which reads model
 *      weights and prompt tokens) ----
 * Stream `seed`: splitmix64 expands the seed into the state of xoshiro256**.  tmac_synth_uniform
 * writes n uniforms in [0, 1) (the top 53 bits of each output times 2^-53); tmac_synth_normal writes
 * n N(0,1) values, two per Box-Muller pair in double precision (radius sqrt(-2 ln(1 - u1)), angle
 * 2 pi u2; cos then sin), each rounded to fp32.  The benchmark and the parity tests draw their inputs
 * from these streams, so both see the same values.  No context, no GPU. */
int tmac_synth_normal(uint64_t seed, float* out, size_t n);
int tmac_synth_uniform(uint64_t seed, double* out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
