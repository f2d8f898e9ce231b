// attn_args.h -- kernel argument blocks shared by the host layer (tmac_attn.cpp)
// and the gfx950 kernels (attn_kernels.hip).  Every kernel takes one of these
// structs by value as its only argument, so hipModuleLaunchKernel passes a
// single pointer in kernelParams.
#pragma once
#include <stdint.h>

namespace tmac {

constexpr int kHeadDim = 64;        // the reference's flash kernel supports only 64 (kernel_flash_attn.metal:18)
constexpr int kSlotsPerWave = 8;    // 64 lanes = 8 (row, kv-head) slots x 8 dim-lanes
constexpr int kGroupWaves = 8;      // "group" decode kernel: 512 threads per workgroup
constexpr int kPrefetchDepth = 3;   // group kernel: steps of K/V in flight per wave (191 VGPRs at G = 7)
constexpr int kPrefetchDepth16 = 6; // the same for 16-bit caches: half the bytes per step, twice the steps
constexpr int kPrefetchDepthQ8 = 8; // the same for Q8_0 caches (136-byte rows at 2 kv heads)
constexpr int kQ8HeadBytes = 68;    // Q8_0 cache: one (row, kv head) = int8 q[64] + fp16 d0, d1
constexpr int kPageRows = 16;       // paged caches: rows per page
constexpr int kPageShift = 4;       // log2(kPageRows)
constexpr int kMWaves16Host = 4;    // MFMA decode kernel, bf16 / fp16 caches: waves per workgroup
constexpr int kMWavesQ8Host = 8;    // MFMA decode kernel, Q8_0 caches (widening needs 2 waves per SIMD)
constexpr int kHeadWaves = 16;      // "head" decode kernel (short contexts): 1024 threads
constexpr int kHeadPrefetchDepth = 2;
constexpr int kHvWaves = 8;         // split-V head kernel (short contexts): 512 threads
constexpr int kHvDepth = 2;         // split-V head kernel: steps of K/V in flight per wave
constexpr int kHvSplitDefault = 8;  // workgroups per query head, each accumulating 64/8 dims of V
constexpr int kAnyWavesHost = 8;    // any-shape decode kernel (shapes with no compiled kernel): 512 threads
constexpr int kAnyMaxDim = 256;     // any-shape kernel and RoPE: even head_dim up to this
constexpr int kMaxSplits = 256;     // split-KV workgroups per sequence, at most
constexpr int kPartialStride = kHeadDim + 2;  // per (split, head): acc[64], m, l

// RoPE row cache of one device-side position counter: two slots, slot s =
// 32 (cos, sin) pairs at float2 offset 32 s, and at float2 offset 64 the
// slots' tags, int [2][4] = {position, RoPE table address low 32 bits, high
// 32 bits, 0}.  tmac_pos_update writes row p of the table the counter's layer
// steps use into slot p % 2 when it sets the counter to p; a layer kernel at
// position p reads both slots while it reads p and uses the one tagged (p,
// its table) if any.  Tags start at -1.
constexpr int kPosSlotBytes = 1024;
constexpr int kPosSlotBlocks = 64;   // position counters with a row cache per context

// Attention over a KV cache in the reference layout: one row per position,
// row = [n_kv_head][64] fp32 (tmac_gguf.cpp:200-201).
struct DecodeArgs {
    const float* q;          // [n_seq][n_head][64]; layer mode: pre-RoPE q of one token
    const float* k;          // cache / pool base (element type per kernel: fp32, bf16, fp16, Q8_0)
    const float* v;
    float* out;              // [n_seq][n_head][64]
    const int64_t* offsets;  // ragged mode: first row of each sequence in the pool
    const int32_t* lengths;  // ragged mode: rows per sequence
    int64_t seq_stride;      // uniform mode: rows between consecutive sequences
    int n_pos;               // uniform mode: rows attended per sequence (past_len + 1)
    int n_head;
    int n_seq;               // ragged mode: sequences (lengths[] entries)
    int split_len;           // rows per workgroup (multiple of the group's step)
    int n_splits;            // gridDim.x
    float* ws;               // split partials [n_seq][n_splits][n_head][66] (n_splits > 1)
    float qscale;            // log2(e) / sqrt(head_dim): softmax runs in base 2
    int rot_mul;             // workgroup w starts its step sequence w*rot_mul steps in (HBM channel spread)
    int blocked;             // group kernel: 1 = each wave streams a contiguous run of steps
    // layer mode (RoPE + cache write + attention in one launch)
    const float* k_new;      // [n_kv_head][64] pre-RoPE
    const float* v_new;      // [n_kv_head][64]
    float* k_out;            // layer cache written at row pos (same memory as k)
    float* v_out;
    const float2* rope_cs;   // [rope_rows][32] (cos, sin) of pos*theta_j
    const int* pos_dev;      // device-side position (graph replay); null -> pos_host
    // With pos_dev: this position counter's cache of RoPE rows (kPosSlotBytes,
    // layout below), so the row of the step's position can be read without
    // waiting for the position; null -> the row is read after the position.
    float2* pos_slots;
    int pos_host;
    int rope_rows;
    int capacity;            // rows in the layer cache (paged layer mode: max_pages * kPageRows)
    int* err;                // device error word (bit 0: position out of range, bit 1: length above
                             // the launch's max_len, bit 2: block-table entry outside the pool)
    // paged modes: the caches are pools of kPageRows-row pages
    const int32_t* block_table;  // [n_seq][max_pages]: pool page of each sequence's logical page
    const int32_t* positions;    // paged layer mode: [n_seq] position of each sequence's new token
    int max_pages;
    int n_pages;                 // pages in each pool
    // stream-K ragged decode: per sequence (first workspace slot, slots used),
    // and the launch's max_len (longer sequences give NaN and error bit 1)
    int32_t* seg_meta;
    int sk_max_len;
    // any-shape kernel (shapes without a compiled kernel): runtime kv heads and head_dim
    int n_kv_head;
    int head_dim;
};

// Chunked causal prefill: query i of sequence s sits at absolute position
// prefix_len + i and attends cache rows 0..prefix_len + i of that sequence.
struct PrefillArgs {
    const float* q;          // [n_seq][n_q][n_head][64]
    const float* k;          // sequence s starts at row s * seq_stride; row = [n_kv_head][64]
    const float* v;
    float* out;              // [n_seq][n_q][n_head][64]
    int64_t seq_stride;
    int n_q;
    int prefix_len;
    int n_qblk;              // ceil(n_q / kPrefillQueries); attention grid = n_qblk * n_kv_head * n_seq
    float qscale;            // log2(e) / sqrt(head_dim)
    uint16_t* packed;        // bf16 tiles [n_seq][n_kv_head][n_tp][K tile, V^T tile] (64 x 64 each)
    int n_tp;                // tiles per (sequence, kv head): ceil(rows / 64) rounded up to a stage
    int n_rows;              // pack: rows row_lo .. n_rows - 1 are written; other rows keep their contents
    int tile0;               // pack: first tile of every (sequence, kv head) this launch packs
    int n_tpp;               // pack: tiles per (sequence, kv head) this launch packs
    // paged caches: k / v are pools of n_pages kPageRows-row pages, sequence s's
    // row r in pool page block_table[s][r / kPageRows] (seq_stride unused)
    const int32_t* block_table;
    int max_pages;
    int n_pages;
    int* err;                // bit 2: a block-table entry outside the pool (clamped)
    int row_lo;              // pack: first row written
};
constexpr int kPrefillQueries = 16;  // queries per workgroup (one MFMA column block)
constexpr int kPrefillKeys = 64;     // keys per tile
constexpr int kPrefillTileElems = 2 * 64 * 64;  // bf16 per packed tile: K [key][dim], then V^T [dim][key]
constexpr int kPrefillStageTiles = 4;           // tiles per LDS stage (two per wave and head pair)
constexpr int kPrefillWaves = 8;     // waves per workgroup: 4 head pairs x 2 stage halves

struct RopeArgs {
    float* x;                // n_rows rows of [n_heads][head_dim], rotated in place; row r at x + r * row_stride
    const float2* rope_cs;   // [rope_rows][head_dim / 2]
    const int* pos_dev;      // position of row 0 (device; null: pos_host); row r sits at position + r
    int pos_host;
    int n_heads;
    int rope_rows;
    int* err;
    int n_rows;
    int64_t row_stride;      // floats between rows
    int head_dim;            // even; cos/sin table rows hold head_dim / 2 pairs
};

struct CopyArgs {
    float* dst;
    const float* src;
    int n;
    int add;                 // 0: dst = src (elem_op 2), 1: dst += src (elem_op 0)
};

// fp32 -> 16-bit cache values (round to nearest even): dst[i] = T(src[i]).
struct CvtArgs {
    const float* src;
    void* dst;
    int64_t n;
    int dtype;               // 1: bf16, 2: fp16 (tmac_cvt16; tmac_cvt_q8 ignores it)
};

// QKV projection of one layer: y[s] = W[s] x (+ bias[s]) for s = q, k, v.
// W[s] is rows[s] rows of cols / 32 blocks; q and k are Q5_0, v is Q8_0 when
// v_is_q8, else Q5_0.  A null bias is absent.
struct QkvArgs {
    const uint8_t* w[3];
    const float* x;          // [cols], 16-byte aligned
    const float* bias[3];
    float* y[3];
    int rows[3];
    int cols;
    int v_is_q8;
};
constexpr int kQkvWaves = 4;         // output rows per workgroup (one wave each)

// y = W x (+ bias) for K-quant weights: rows of cols / 256 super-blocks, Q4_K
// (type 12, 144 bytes) or Q6_K (type 14, 210 bytes).  bias may equal y (the
// residual form y += W x).
struct KqArgs {
    const uint8_t* w;
    const float* x;          // [cols], 16-byte aligned
    const float* bias;
    float* y;
    int rows;
    int cols;
    int type;
};

struct PosArgs {
    int* pos;
    int value;
    int add;                 // 0: *pos = value; 1: *pos += value
    // the counter's RoPE row cache and the table its layer steps use (null: none)
    float2* slots;
    const float2* rope_cs;
    int rope_rows;
};

}  // namespace tmac
