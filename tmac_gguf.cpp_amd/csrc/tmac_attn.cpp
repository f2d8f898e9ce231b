// tmac_attn.cpp -- host layer of libtmac_attn.so: the C ABI declared in
// include/tmac_attn.h, implemented over the HIP runtime.
//
// Replaces the reference's Metal backend for the attention path:
//   init / shutdown              metal_backend.cpp:21-89, metal_backend.hpp:519-520
//   attention_op / rope_op / elem_op   metal_backend.hpp:354-453
//   metal_batch_begin / _end     metal_backend.hpp:114-122, 176-190 (-> hipGraph capture)
// The gfx950 code object (attn_kernels.hip) is linked into this library as
// bytes and loaded with hipModuleLoadData; kernels launch with
// hipModuleLaunchKernel.  There is no CPU fallback: without a gfx950 device
// tmac_init fails and every other entry point reports TMAC_ERR_NOT_INITIALIZED.
#include "tmac_attn.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <numeric>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "attn_args.h"

// The gfx950 code objects, one per kernel part (code_object.S).
constexpr int kCodeParts = 4;
extern "C" const unsigned char* const tmac_attn_code_objects[kCodeParts];
extern "C" const uint64_t tmac_attn_code_object_sizes[kCodeParts];
// tmac_scratch.hip: the device address of the fixed scratch array on `device` (the current device).
extern "C" int tmac_scratch_setup(int device, void** ptr);

using tmac::CopyArgs;
using tmac::CvtArgs;
using tmac::DecodeArgs;
using tmac::PrefillArgs;
using tmac::kPrefillKeys;
using tmac::kPrefillQueries;
using tmac::kPrefillStageTiles;
using tmac::kPrefillTileElems;
using tmac::kPrefillWaves;
using tmac::PosArgs;
using tmac::KqArgs;
using tmac::QkvArgs;
using tmac::kQkvWaves;
using tmac::RopeArgs;
using tmac::kHeadDim;
using tmac::kAnyMaxDim;
using tmac::kPartialStride;
using tmac::kGroupWaves;
using tmac::kHeadWaves;
using tmac::kMaxSplits;
using tmac::kSlotsPerWave;
using tmac::kPageRows;

namespace {

constexpr int kHeadMaxRows = 1024;  // automatic choice: head kernel up to this many rows
// (G = n_head / n_kv_head, KV = n_kv_head) pairs compiled into the code object.
constexpr int kShapes[][2] = {{7, 2}, {1, 1}, {1, 2}, {2, 2}, {4, 2}, {4, 4}, {8, 1}};
enum { kModeUniform = 0, kModeRagged = 1, kModeLayer = 2 };
enum { kPagedDecode = 0, kPagedLayer = 1 };
constexpr int kNarrowTypes = 3;  // TMAC_KV_BF16, TMAC_KV_F16, TMAC_KV_Q8_0 (index kv_dtype - 1)
const char* const kTypeName[4] = {"f32", "bf16", "f16", "q8"};  // by kv_dtype


struct RopeTable {
    int head_dim;
    uint32_t base_bits;
    float2* dev;
    int rows;
};

}  // namespace

struct tmac_graph {
    hipGraphExec_t exec = nullptr;
    tmac_context* owner = nullptr;  // counted in owner->live_graphs while exec is set
};

struct tmac_model {
    struct Entry {
        std::string name;
        uint64_t rows = 0, cols = 0, n_bytes = 0;
        uint32_t type = 0;
        size_t offset = 0;  // into blob, 256-byte aligned
    };
    std::vector<Entry> tensors;
    std::unordered_map<std::string, size_t> index;  // name -> first tensor of that name
    uint8_t* blob = nullptr;                        // device allocation, or 256-byte aligned inside host
    std::unique_ptr<uint8_t[]> host;
    size_t bytes = 0;
    bool on_device = false;
};

struct tmac_context {
    int device = -1;
    int n_cu = 0;
    hipModule_t modules[kCodeParts] = {};
    std::map<std::pair<int, int>, hipFunction_t> decode[3];   // group kernel, by mode, (G, KV)
    std::map<std::pair<int, int>, hipFunction_t> decode4[3];  // group kernel with 4-wave workgroups
    std::map<std::pair<int, int>, hipFunction_t> head[3];     // head kernel (16 waves), same keys
    std::map<std::pair<int, int>, hipFunction_t> head8[3];    // head kernel, 8 waves
    std::map<std::pair<int, int>, hipFunction_t> head4[3];    // head kernel, 4 waves
    std::map<std::pair<int, int>, hipFunction_t> hv[4][3];    // split-V head kernel by log2(V split), same keys
    std::map<std::pair<int, int>, hipFunction_t> combine[3];  // split merge, same keys
    std::map<std::pair<int, int>, hipFunction_t> decode_n[kNarrowTypes][3];  // bf16 / fp16 / Q8_0 caches: group kernel
    std::map<std::pair<int, int>, hipFunction_t> head_n[kNarrowTypes][3];    // the same: head kernel, 8 waves
    std::map<std::pair<int, int>, hipFunction_t> paged[4][2];  // paged caches by kv_dtype: decode, layer step
    std::map<std::pair<int, int>, hipFunction_t> combine_p[2];  // split merge of the paged modes
    std::map<std::pair<int, int>, hipFunction_t> decode_sk, combine_sk;  // stream-K ragged decode (fp32)
    std::map<std::pair<int, int>, hipFunction_t> decode_sk_p;             // the same over paged caches
    std::map<std::pair<int, int>, hipFunction_t> layer_sk_p, combine_sk_l;  // stream-K paged layer step (fp32)
    std::map<std::pair<int, int>, hipFunction_t> mdecode_sk[kNarrowTypes][2];  // MFMA stream-K: ragged, paged
    // MFMA decode (bf16, fp16, Q8_0): uniform, ragged, paged, layer, paged layer
    std::map<std::pair<int, int>, hipFunction_t> mdecode[kNarrowTypes][5];
    std::map<std::pair<int, int>, hipFunction_t> prefill;     // chunked prefill, (G, KV)
    std::map<int, hipFunction_t> prefill_pack[2][4];          // prefill tile packing: [paged][cache type], by KV
    hipFunction_t any[3] = {};  // any-shape decode kernel by mode (shapes with no compiled kernel)
    hipFunction_t k_rope = nullptr, k_copy = nullptr, k_pos = nullptr, k_qkv = nullptr, k_cvt16 = nullptr,
                  k_kq = nullptr, k_cvt_q8 = nullptr;
    float* ws = nullptr;
    size_t ws_floats = 0;
    int* err = nullptr;
    // The library's own copies and fills (tables, tags, the error word) go on
    // this non-blocking stream and wait for it alone: on this runtime a
    // legacy-stream copy or a device-wide synchronize issued while a stream of
    // another thread is capturing fails and ends that capture.
    hipStream_t aux = nullptr;
    // RoPE row caches of the device-side position counters the layer entry
    // points have seen (kPosSlotBlocks blocks of kPosSlotBytes, allocated and
    // tagged empty at init); counters past the last block run without one.
    char* pos_slot_pool = nullptr;
    std::map<const int*, int> pos_slot_of;
    // the RoPE table (device rows, row count) of each counter's latest layer step
    std::map<const int*, std::pair<const float2*, int>> pos_table_of;
    std::vector<RopeTable> rope;
    // Executable step graphs alive on this context.  A captured graph keeps
    // the workspace and RoPE-table addresses it was recorded with, so while
    // any graph is alive a buffer replaced by a larger one is retired (kept
    // allocated) instead of freed; retired buffers are freed when the last
    // graph is destroyed, or at shutdown.
    int live_graphs = 0;
    std::vector<void*> retired;
    // Device address of the fixed scratch array on this context's device
    // (TMAC_SCRATCH_BYTES), resolved once at init.
    float* scratch = nullptr;
    // Set only for the duration of a call of an entry point that allocates
    // nothing: the workspace is then this fixed buffer of fixed_floats floats
    // instead of ws, and nothing grows.
    float* fixed_ws = nullptr;
    size_t fixed_floats = 0;
    std::vector<tmac_graph*> graphs;  // the live graphs, detached from the context at shutdown
    int64_t opt_split_len = 0;
    int64_t opt_target_groups = 0;
    int64_t opt_kernel = TMAC_KERNEL_AUTO;
    int64_t opt_rot_mul = 0;
    int64_t opt_head_waves = 8;
    int64_t opt_blocked = 0;
    int64_t opt_group_waves = 0;  // 0: automatic (auto_group_waves)
    int64_t opt_mfma = 1;
    int64_t opt_stream_k = 1;
    int64_t opt_hv_split = tmac::kHvSplitDefault;
    std::string last_error;
    char device_name[256] = {0};
};

namespace {

int fail(tmac_context* ctx, int code, const std::string& msg) {
    if (ctx) ctx->last_error = msg;
    return code;
}

int hip_fail(tmac_context* ctx, hipError_t e, const char* what) {
    if (ctx) ctx->last_error = std::string(what) + ": " + hipGetErrorString(e);
    return TMAC_ERR_HIP_BASE + (int)e;
}

#define HIP_TRY(ctx, expr)                                   \
    do {                                                     \
        hipError_t e_ = (expr);                              \
        if (e_ != hipSuccess) return hip_fail(ctx, e_, #expr); \
    } while (0)

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_ctx(tmac_context* ctx) {
    if (!ctx || !ctx->modules[0]) return TMAC_ERR_NOT_INITIALIZED;
    return TMAC_OK;
}

int set_device(tmac_context* ctx) {
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    return TMAC_OK;
}

// Looks a kernel up in whichever code object part holds it.
hipError_t get_function(tmac_context* ctx, hipFunction_t* f, const char* name) {
    for (auto m : ctx->modules)
        if (m && hipModuleGetFunction(f, m, name) == hipSuccess) return hipSuccess;
    (void)hipGetLastError();
    return hipErrorNotFound;
}

bool capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) return false;
    return st != hipStreamCaptureStatusNone;
}

// Step captures (tmac_step_begin .. tmac_step_end) in progress in any context
// of the process.  While one is, no context synchronizes the whole device (a
// device-wide synchronize from another thread fails and ends that capture):
// buffers a growth replaces are retired instead of freed after a synchronize,
// and the error check reads the error word without one.
std::atomic<int> g_captures{0};

// Synchronizes the context's device when no step capture is in progress;
// true when the device is then idle.
bool quiesce(tmac_context* ctx) {
    if (g_captures.load() != 0) return false;
    (void)hipSetDevice(ctx->device);
    return hipDeviceSynchronize() == hipSuccess;
}

hipError_t aux_fill(tmac_context* ctx, void* p, int value, size_t bytes) {
    hipError_t e = hipMemsetAsync(p, value, bytes, ctx->aux);
    return e != hipSuccess ? e : hipStreamSynchronize(ctx->aux);
}

hipError_t aux_copy(tmac_context* ctx, void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
    hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, ctx->aux);
    return e != hipSuccess ? e : hipStreamSynchronize(ctx->aux);
}

struct Kernels {
    hipFunction_t group = nullptr, head = nullptr, combine = nullptr;
    hipFunction_t hv = nullptr;      // short-context split-V head kernel (fp32 caches, not paged)
    hipFunction_t any = nullptr;     // any-shape kernel: a shape with no compiled kernel (fp32, not paged)
    int hv_split = 1;
    hipFunction_t group4 = nullptr;  // 4-wave group kernel when the size is chosen per call (fp32 caches)
    int head_waves = 16;
    int group_waves = 8;
};

// Validates the attention shape shared by every decode entry point and picks
// the kernels for cache element type `dt` (TMAC_KV_F32 / _BF16 / _F16 / _Q8_0;
// the narrow caches use the default 8-wave group and head kernels).  paged:
// -1, or kPagedDecode / kPagedLayer for the paged kernels (group kernel only).
int check_shape(tmac_context* ctx, int n_head, int n_kv_head, int head_dim, Kernels* k, int mode,
                int dt = TMAC_KV_F32, int paged = -1) {
    if (dt != TMAC_KV_F32 && dt != TMAC_KV_BF16 && dt != TMAC_KV_F16 && dt != TMAC_KV_Q8_0)
        return fail(ctx, TMAC_ERR_INVALID_ARG,
                    "kv_dtype must be TMAC_KV_F32, TMAC_KV_BF16, TMAC_KV_F16 or TMAC_KV_Q8_0");
    if (n_head <= 0 || n_kv_head <= 0 || n_head % n_kv_head != 0)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "n_head must be a positive multiple of n_kv_head");
    const int g = n_head / n_kv_head;
    auto it = ctx->decode[mode].find({g, n_kv_head});
    if (head_dim != kHeadDim || it == ctx->decode[mode].end()) {
        // No compiled kernel for the shape: fp32, unpaged caches take the any-shape kernel (the
        // reference's kernel_attn fallback: any group, head_dim even and at most kAnyMaxDim here).
        if (dt == TMAC_KV_F32 && paged < 0 && head_dim >= 2 && head_dim <= kAnyMaxDim && head_dim % 2 == 0) {
            if (k) {
                *k = Kernels{};
                k->any = ctx->any[mode];
            }
            return TMAC_OK;
        }
        if (head_dim != kHeadDim)
            return fail(ctx, TMAC_ERR_UNSUPPORTED,
                        "head_dim " + std::to_string(head_dim) +
                            ": only 64 on this entry point and cache type (fp32 attention, layer and batched "
                            "decode also take even head_dim up to 256)");
        return fail(ctx, TMAC_ERR_UNSUPPORTED,
                    "no kernel for n_head/n_kv_head = " + std::to_string(g) + ", n_kv_head = " +
                        std::to_string(n_kv_head) + " on this entry point and cache type");
    }
    if (k) {
        k->group_waves = ctx->opt_group_waves == 4 ? 4 : 8;
        k->group = k->group_waves == 4 ? ctx->decode4[mode].at({g, n_kv_head}) : it->second;
        if (ctx->opt_group_waves == 0) k->group4 = ctx->decode4[mode].at({g, n_kv_head});
        k->head_waves = (int)ctx->opt_head_waves;
        k->head = (k->head_waves == 8 ? ctx->head8 : k->head_waves == 4 ? ctx->head4 : ctx->head)[mode].at({g, n_kv_head});
        k->combine = ctx->combine[mode].at({g, n_kv_head});
        k->hv_split = (int)ctx->opt_hv_split;
        k->hv = ctx->hv[__builtin_ctz(k->hv_split)][mode].at({g, n_kv_head});
        if (dt != TMAC_KV_F32) {
            k->hv = nullptr;
            k->group4 = nullptr;
            k->group_waves = 8;
            k->group = ctx->decode_n[dt - 1][mode].at({g, n_kv_head});
            k->head_waves = 8;
            k->head = ctx->head_n[dt - 1][mode].at({g, n_kv_head});
        }
        if (paged >= 0) {
            k->hv = nullptr;
            k->group4 = nullptr;
            k->group_waves = kGroupWaves;
            k->group = ctx->paged[dt][paged].at({g, n_kv_head});
            k->head = nullptr;
            k->combine = ctx->combine_p[paged].at({g, n_kv_head});
        }
        // Narrow caches: the group kernel is the MFMA kernel where one is built for the shape.
        const int mm = paged == kPagedDecode ? 2 : paged == kPagedLayer ? 4 : mode == kModeLayer ? 3 : mode;
        if (dt != TMAC_KV_F32 && ctx->opt_mfma) {
            auto& tab = ctx->mdecode[dt - 1][mm];
            auto f = tab.find({g, n_kv_head});
            if (f != tab.end()) {
                k->group = f->second;
                k->group_waves = dt == TMAC_KV_Q8_0 ? tmac::kMWavesQ8Host : tmac::kMWaves16Host;
            }
        }
    }
    return TMAC_OK;
}

// Group kernel: rows per workgroup, a multiple of one round of steps over the
// workgroup (kGroupWaves steps of 8/n_kv_head rows).  Aims for `target`
// workgroups (one per CU by default: a 512-thread workgroup at 2 waves per
// SIMD fills a CU) without going below one round per workgroup, and keeps at
// most kMaxSplits splits per sequence.
// With `total_rows` (ragged batches: the sum of all lengths, when the caller
// knows it) the split length is total/target instead, so the workgroups that
// actually have rows come close to one per CU whatever the length mix.
void choose_split(const tmac_context* ctx, int waves, int n_seq, int n_pos, int n_kv_head, int* split_len,
                  int* n_splits, int64_t total_rows = 0, int align = 1) {
    // `align`: split lengths are also a multiple of it (paged caches: the
    // 16-row page, which the MFMA decode's tiles and the group kernel's steps
    // must not straddle).
    const int round = std::lcm(waves * (kSlotsPerWave / n_kv_head), align);
    const int rounds = (n_pos + round - 1) / round;
    int len;
    const int64_t target_groups = ctx->opt_target_groups > 0 ? ctx->opt_target_groups : (int64_t)ctx->n_cu;
    if (ctx->opt_split_len > 0) {
        len = (int)(((ctx->opt_split_len + round - 1) / round) * round);
    } else if (total_rows > 0 && target_groups > n_seq) {
        const int64_t per = (total_rows + (target_groups - n_seq) - 1) / (target_groups - n_seq);
        len = (int)std::min<int64_t>(((per + round - 1) / round) * round, (int64_t)rounds * round);
    } else {
        int64_t want = (target_groups + n_seq - 1) / (n_seq > 0 ? n_seq : 1);
        if (want < 1) want = 1;
        if (want > rounds) want = rounds;
        const int64_t per = (rounds + want - 1) / want;
        len = (int)(per * round);
    }
    if (len < round) len = round;
    while ((n_pos + (int64_t)len - 1) / len > kMaxSplits) len += round;
    *split_len = len;
    *n_splits = (n_pos + len - 1) / len;
    if (*n_splits < 1) *n_splits = 1;
}

// fp32 group kernel size when TMAC_OPT_GROUP_WAVES is 0 (automatic).  Four
// waves per workgroup give each wave twice the run of rows and halve the
// cross-wave merge: config 3 164 vs 166 us, config 4 60.6 vs 63.7 us,
// 64 x 4096 rows 49 vs 52 us.  Unless a split would then hold fewer than
// kAuto4MinRows rows (one sequence over all CUs: 16-row splits, twice the
// partials to combine; 1 x 4096 rows 26 vs 20 us), where 8 waves are used.
constexpr int kAuto4MinRows = 64;
int auto_group_waves(const tmac_context* ctx, int n_seq, int rows, int n_kv_head, int64_t total_rows) {
    int len = 0, n_splits = 0;
    choose_split(ctx, 4, n_seq, rows, n_kv_head, &len, &n_splits, total_rows);
    return len >= kAuto4MinRows ? 4 : 8;
}

// One workgroup per query head (the row kernel, or the head kernel) for short
// contexts that would leave most CUs idle otherwise.
bool use_head_kernel(const tmac_context* ctx, int n_seq, int n_head, int rows) {
    if (ctx->opt_kernel == TMAC_KERNEL_HEAD || ctx->opt_kernel == TMAC_KERNEL_HEADV) return true;
    if (ctx->opt_kernel == TMAC_KERNEL_GROUP) return false;
    return (int64_t)n_seq * n_head < 2LL * ctx->n_cu && rows <= kHeadMaxRows;
}

// The split-KV workspace of the current call (valid after ensure_workspace).
float* workspace(const tmac_context* ctx) { return ctx->fixed_ws ? ctx->fixed_ws : ctx->ws; }

// Makes the fixed scratch buffer the workspace for one call.
struct FixedWorkspace {
    tmac_context* ctx;
    FixedWorkspace(tmac_context* c, float* p, size_t floats) : ctx(c) {
        ctx->fixed_ws = p;
        ctx->fixed_floats = floats;
    }
    ~FixedWorkspace() {
        ctx->fixed_ws = nullptr;
        ctx->fixed_floats = 0;
    }
};

// Frees a device buffer the context no longer uses (`idle`: the device was
// synchronized, so no kernel still reads it), or retires it while a step graph
// that may have recorded its address is alive or the device could not be
// synchronized.
void release_buffer(tmac_context* ctx, void* p, bool idle) {
    if (!p) return;
    if (ctx->live_graphs > 0 || !idle)
        ctx->retired.push_back(p);
    else
        (void)hipFree(p);
}

// Drops a graph from its context's live count (its executable is gone).
void forget_graph(tmac_graph* g) {
    tmac_context* ctx = g->owner;
    g->owner = nullptr;
    if (!ctx) return;
    ctx->live_graphs--;
    auto it = std::find(ctx->graphs.begin(), ctx->graphs.end(), g);
    if (it != ctx->graphs.end()) ctx->graphs.erase(it);
}

// Frees the retired buffers once the device can be synchronized (otherwise
// they wait for a later call, or shutdown).  A freed RoPE table's address may
// come back for another table, so every row-cache tag is cleared with them.
void free_retired(tmac_context* ctx) {
    if (ctx->retired.empty() || !quiesce(ctx)) return;
    for (void* p : ctx->retired) (void)hipFree(p);
    ctx->retired.clear();
    (void)aux_fill(ctx, ctx->pos_slot_pool, 0xFF, (size_t)tmac::kPosSlotBlocks * tmac::kPosSlotBytes);
}

int ensure_workspace(tmac_context* ctx, hipStream_t stream, size_t floats) {
    if (ctx->fixed_ws) {
        if (floats <= ctx->fixed_floats) return TMAC_OK;
        return fail(ctx, TMAC_ERR_CAPACITY,
                    "the call needs " + std::to_string(floats * sizeof(float)) +
                        " bytes of split-KV workspace, more than the fixed scratch buffer's " +
                        std::to_string(ctx->fixed_floats * sizeof(float)) + " (TMAC_SCRATCH_BYTES)");
    }
    if (floats <= ctx->ws_floats) return TMAC_OK;
    if (capturing(stream))
        return fail(ctx, TMAC_ERR_CAPTURE,
                    "split-KV workspace must grow but the stream is capturing; run the same shape once "
                    "before capture");
    const bool idle = quiesce(ctx);
    size_t n = ctx->ws_floats ? ctx->ws_floats : (1u << 20);
    while (n < floats) n *= 2;
    float* p = nullptr;
    HIP_TRY(ctx, hipMalloc(&p, n * sizeof(float)));
    release_buffer(ctx, ctx->ws, idle);
    ctx->ws = p;
    ctx->ws_floats = n;
    return TMAC_OK;
}

uint32_t float_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

// cos/sin of pos*theta_j exactly as tmac_gguf.cpp:994-997 computes them
// (fp32 theta = 1/powf(base, d/head_dim), fp32 angle = pos*theta, libm
// cosf/sinf); built on the host so the device rotation is bit-identical to
// the reference's CPU path.  This file is compiled with -ffp-contract=off
// -fno-builtin so that nothing is fused or merged into sincosf.
int rope_table(tmac_context* ctx, hipStream_t stream, int head_dim, float base, int need_rows,
               const RopeTable** out) {
    RopeTable* found = nullptr;
    for (auto& t : ctx->rope)
        if (t.head_dim == head_dim && t.base_bits == float_bits(base)) found = &t;
    if (found && found->rows >= need_rows) {
        *out = found;
        return TMAC_OK;
    }
    if (capturing(stream))
        return fail(ctx, TMAC_ERR_CAPTURE,
                    "RoPE table must grow but the stream is capturing; call tmac_rope_prepare first");
    int rows = found ? found->rows : 0;
    int new_rows = rows > 0 ? rows : 4096;
    while (new_rows < need_rows) {
        if (new_rows > INT_MAX / 2) { new_rows = need_rows; break; }
        new_rows *= 2;
    }
    const int pairs = head_dim / 2;
    std::vector<float2> host((size_t)new_rows * pairs);
    for (int pos = 0; pos < new_rows; pos++) {
        for (int d = 0; d < head_dim; d += 2) {
            float theta = 1.0f / powf(base, (float)d / head_dim);
            float freq = pos * theta;
            host[(size_t)pos * pairs + d / 2] = make_float2(cosf(freq), sinf(freq));
        }
    }
    float2* dev = nullptr;
    const bool idle = quiesce(ctx);
    HIP_TRY(ctx, hipMalloc(&dev, host.size() * sizeof(float2)));
    HIP_TRY(ctx, aux_copy(ctx, dev, host.data(), host.size() * sizeof(float2), hipMemcpyHostToDevice));
    // The position counters' RoPE row caches are tagged with table addresses,
    // and a new table may reuse a freed one's address: with the device idle
    // every tag is cleared.  Otherwise no table is freed (the old one is
    // retired), so no address comes back and the tags stay (kernels may be
    // reading them).
    if (idle)
        HIP_TRY(ctx, aux_fill(ctx, ctx->pos_slot_pool, 0xFF, (size_t)tmac::kPosSlotBlocks * tmac::kPosSlotBytes));
    if (found) {
        // counters whose row caches tmac_pos_update refreshes from this table
        for (auto& pt : ctx->pos_table_of)
            if (pt.second.first == found->dev) pt.second = {dev, new_rows};
        release_buffer(ctx, found->dev, idle);
        found->dev = dev;
        found->rows = new_rows;
    } else {
        ctx->rope.push_back(RopeTable{head_dim, float_bits(base), dev, new_rows});
        found = &ctx->rope.back();
    }
    *out = found;
    return TMAC_OK;
}

int launch(tmac_context* ctx, hipFunction_t f, unsigned gx, unsigned gy, unsigned block, hipStream_t stream,
           void* args, unsigned gz = 1) {
    void* params[] = {args};
    HIP_TRY(ctx, hipModuleLaunchKernel(f, gx, gy, gz, block, 1, 1, 0, stream, params, nullptr));
    return TMAC_OK;
}

const float kQScale = (float)(1.4426950408889634 / 8.0);  // log2(e) / sqrt(64)

// Common launch of a decode-family kernel, plus the split merge when the
// rows are spread over more than one workgroup per sequence.
int run_decode(tmac_context* ctx, hipStream_t stream, const Kernels& k, DecodeArgs& a, int n_seq,
               int grid_rows, int n_kv_head, int64_t total_rows = 0) {
    a.qscale = kQScale;
    a.rot_mul = (int)ctx->opt_rot_mul;
    a.blocked = (int)ctx->opt_blocked;
    a.err = ctx->err;
    if (n_seq > 65535) return fail(ctx, TMAC_ERR_INVALID_ARG, "n_seq exceeds 65535");
    if (k.any) {  // one workgroup per (query head, sequence), no split
        a.split_len = grid_rows;
        a.n_splits = 1;
        a.ws = nullptr;
        a.n_kv_head = n_kv_head;
        return launch(ctx, k.any, (unsigned)a.n_head, (unsigned)n_seq, tmac::kAnyWavesHost * 64, stream, &a);
    }
    const bool unit_grid = a.lengths || a.positions;  // ragged and paged modes
    if (k.head && use_head_kernel(ctx, n_seq, a.n_head, grid_rows)) {
        a.split_len = grid_rows;
        a.n_splits = 1;
        a.ws = nullptr;
        if (k.hv && ctx->opt_kernel != TMAC_KERNEL_HEAD)
            return launch(ctx, k.hv, (unsigned)(a.n_head * k.hv_split), (unsigned)n_seq, tmac::kHvWaves * 64, stream,
                          &a);
        return launch(ctx, k.head, (unsigned)a.n_head, (unsigned)n_seq, k.head_waves * 64, stream, &a);
    }
    hipFunction_t group = k.group;
    int waves = k.group_waves;
    if (k.group4 && auto_group_waves(ctx, n_seq, grid_rows, n_kv_head, total_rows) == 4) {
        group = k.group4;
        waves = 4;
    }
    int split_len = 0, n_splits = 0;
    choose_split(ctx, waves, n_seq, grid_rows, n_kv_head, &split_len, &n_splits, total_rows,
                 a.block_table ? kPageRows : 1);
    a.split_len = split_len;
    a.n_splits = n_splits;
    if (n_splits > 1) {
        const size_t need = (size_t)n_seq * n_splits * a.n_head * kPartialStride;
        int rc = ensure_workspace(ctx, stream, need);
        if (rc) return rc;
        a.ws = workspace(ctx);
    } else {
        a.ws = nullptr;
    }
    a.n_seq = n_seq;
    int rc;
    if (unit_grid) {  // flat unit grid, n_seq * n_splits bounds the unit count
        const int64_t units = (int64_t)n_seq * n_splits;
        if (units > INT_MAX) return fail(ctx, TMAC_ERR_INVALID_ARG, "decode_ragged: too many splits");
        rc = launch(ctx, group, (unsigned)units, 1, waves * 64, stream, &a);
    } else {
        rc = launch(ctx, group, (unsigned)n_splits, (unsigned)n_seq, waves * 64, stream, &a);
    }
    if (rc || n_splits == 1) return rc;
    return launch(ctx, k.combine, (unsigned)a.n_head, (unsigned)n_seq, 64, stream, &a);
}

// Schedule of the ragged and paged decode and of the paged layer step: the
// unit grid (run_decode) or stream-K (run_decode_sk).
// fp32 ragged decode: stream-K pays a pipeline
// restart and a merge at every sequence change inside a range, so it wins
// while ranges hold few sequences, and again at many sequences, where the
// unit grid's serial scan of the lengths dominates.  Measured with lengths
// uniform in 1..L (unit grid -> stream-K, us): 128 x 8192: 108 -> 93;
// 256 x 4096: 107 -> 96; 384 x 2048: 97 -> 81; 1024 x 512: 63 -> 83;
// 1536 x 1024: 148 -> 160; 2048 x 1024: 198 -> 214; 3000 x 40: 180 -> 85;
// 4096 x 256: 194 -> 178; 20000 x U[0, 12]: 3700 -> 350; 60000 x U[0, 12]:
// 29600 -> 1062 (every unit-grid workgroup scans the lengths up to its
// unit, so that grid's cost grows with the square of the sequence count).
// Fewer sequences split well on the unit grid:
// 16 x 32768 59.1 -> 59.6, 64 x 16384 95.6 -> 96.7, 256 x 4096 equal
// lengths 159.1 -> 160.4.
// Paged caches (the unit grid there runs 8-wave workgroups): stream-K wins
// from half a sequence per CU on: 128 x 8192 111 -> 96, 384 x 2048 99 -> 83,
// 1024 x 512 79 -> 73, 3000 x 40 178 -> 84, 4096 x 256 320 -> 178; but
// 16 x 32768 60.4 -> 62.6.
// MFMA decode (bf16 / fp16 / Q8_0 caches, ragged or paged): a segment's setup
// (query split into parts, tiles spread over 8 waves, LDS merge) is heavier,
// so only the many-sequence case gains: bf16 3000 x 40 144 -> 105, Q8_0
// 154 -> 120; but bf16 384 x 2048 53 -> 64, 1024 x 512 54 -> 81, 2048 x 512
// 119 -> 124, Q8_0 1024 x 512 61 -> 81.
// Paged layer step (fp32): the unit grid has no row-count hint there and
// sizes its splits from max_len, so stream-K wins from few sequences on:
// positions U[0, L): 16 x 32768 56.8 -> 49.8, 64 x 16384 106 -> 89,
// 128 x 8192 109 -> 98, 256 x 4096 113 -> 107, 384 x 2048 99 -> 92,
// 3000 x 40 184 -> 97; but 1024 x 512 82 -> 90.
enum SkKind { kSkF32Ragged, kSkF32Paged, kSkF32Layer, kSkMfma };
bool use_stream_k(const tmac_context* ctx, int n_seq, SkKind kind) {
    if (ctx->opt_stream_k == 0) return false;
    if (ctx->opt_stream_k == 2) return true;
    const int64_t n2 = 2 * (int64_t)n_seq;
    if (kind == kSkF32Paged) return n2 >= ctx->n_cu;
    const bool many = n_seq > 10 * ctx->n_cu;
    if (kind == kSkMfma) return many;
    if (kind == kSkF32Layer) return n_seq <= 2 * ctx->n_cu || many;
    return (n2 >= ctx->n_cu && n2 <= 3 * (int64_t)ctx->n_cu) || many;
}

// Stream-K kernel for a ragged (paged = false) or paged batch of cache type
// dt and its block size, or null when the schedule does not apply.
hipFunction_t stream_k_kernel(const tmac_context* ctx, int dt, bool paged, int n_seq, int n_head, int n_kv_head,
                              unsigned* threads) {
    const SkKind kind = dt != TMAC_KV_F32 ? kSkMfma : paged ? kSkF32Paged : kSkF32Ragged;
    if (ctx->opt_split_len != 0 || !use_stream_k(ctx, n_seq, kind)) return nullptr;
    const std::pair<int, int> key{n_head / n_kv_head, n_kv_head};
    if (dt == TMAC_KV_F32) {
        *threads = 256;
        return (paged ? ctx->decode_sk_p : ctx->decode_sk).at(key);
    }
    if (!ctx->opt_mfma) return nullptr;
    const auto& tab = ctx->mdecode_sk[dt - 1][paged ? 1 : 0];
    const auto it = tab.find(key);
    if (it == tab.end()) return nullptr;
    *threads = (dt == TMAC_KV_Q8_0 ? tmac::kMWavesQ8Host : tmac::kMWaves16Host) * 64;
    return it->second;
}

// Stream-K launch (ragged or paged decode on any cache type, fp32 paged
// layer step): the kernel cuts the batch's padded row space into `units`
// equal ranges (one workgroup each, one per CU by default), sized from the
// lengths or positions on the device, so the total_rows hint is not needed
// and graph replays may change them.  The workspace holds units + n_seq
// partial slots whatever the lengths.  The combine launch always follows: it
// merges the sequences spread over several workgroups and writes the outputs
// of empty and over-long ones.
int run_decode_sk(tmac_context* ctx, hipStream_t stream, hipFunction_t sk, unsigned threads, hipFunction_t combine,
                  DecodeArgs& a, int n_seq, int max_len) {
    a.qscale = kQScale;
    a.rot_mul = (int)ctx->opt_rot_mul;
    a.blocked = (int)ctx->opt_blocked;
    a.err = ctx->err;
    a.sk_max_len = max_len;
    if (n_seq > 65535) return fail(ctx, TMAC_ERR_INVALID_ARG, "n_seq exceeds 65535");
    if (max_len > INT_MAX - kPageRows) return fail(ctx, TMAC_ERR_INVALID_ARG, "stream-K decode: max_len too large");
    // One workgroup per CU; two when the sequences outnumber the CUs (more
    // sequence changes per range, whose stalls the second workgroup covers).
    const int64_t auto_units = (int64_t)ctx->n_cu * (n_seq > ctx->n_cu ? 2 : 1);
    const int64_t units = std::min<int64_t>(ctx->opt_target_groups > 0 ? ctx->opt_target_groups : auto_units, 1 << 20);
    const size_t slot_floats = (size_t)a.n_head * kPartialStride;
    const size_t slots = (size_t)units + (size_t)n_seq;
    int rc = ensure_workspace(ctx, stream, slots * slot_floats + 2 * (size_t)n_seq);
    if (rc) return rc;
    a.ws = workspace(ctx);
    a.seg_meta = reinterpret_cast<int32_t*>(a.ws + slots * slot_floats);
    a.split_len = 0;
    a.n_splits = (int)units;
    a.n_seq = n_seq;
    if ((rc = launch(ctx, sk, (unsigned)units, 1, threads, stream, &a))) return rc;
    return launch(ctx, combine, (unsigned)a.n_head, (unsigned)n_seq, 64, stream, &a);
}

}  // namespace

extern "C" {

const char* tmac_status_string(int status) {
    switch (status) {
        case TMAC_OK: return "ok";
        case TMAC_ERR_INVALID_ARG: return "invalid argument";
        case TMAC_ERR_NULL_POINTER: return "null pointer";
        case TMAC_ERR_MISALIGNED: return "pointer not 16-byte aligned";
        case TMAC_ERR_UNSUPPORTED: return "unsupported shape or operation";
        case TMAC_ERR_CAPACITY: return "position or size beyond capacity";
        case TMAC_ERR_NOT_INITIALIZED: return "context not initialized";
        case TMAC_ERR_CAPTURE: return "not allowed while the stream is capturing";
        case TMAC_ERR_DEVICE_FAULT: return "device reported an out-of-range position";
        case TMAC_ERR_NOT_FOUND: return "no tensor of that name";
        case TMAC_ERR_IO: return "weight file missing, truncated or not a TMAC file";
        default: break;
    }
    if (status >= TMAC_ERR_HIP_BASE) return hipGetErrorString((hipError_t)(status - TMAC_ERR_HIP_BASE));
    return "unknown status";
}

const char* tmac_last_error(const tmac_context* ctx) { return ctx ? ctx->last_error.c_str() : ""; }

int tmac_abi_version(void) { return TMAC_ATTN_ABI_VERSION; }

int tmac_init(tmac_context** out, int device) {
    if (!out) return TMAC_ERR_NULL_POINTER;
    *out = nullptr;
    auto* ctx = new tmac_context();
    ctx->device = device;
    int n_dev = 0;
    hipError_t e = hipGetDeviceCount(&n_dev);
    if (e != hipSuccess || n_dev <= device || device < 0) {
        int rc = e != hipSuccess ? hip_fail(ctx, e, "hipGetDeviceCount")
                                 : fail(ctx, TMAC_ERR_INVALID_ARG, "no such device");
        delete ctx;
        return rc;
    }
    auto bail = [&](int rc) {
        if (ctx->aux) (void)hipStreamSynchronize(ctx->aux);
        if (ctx->ws) (void)hipFree(ctx->ws);
        if (ctx->err) (void)hipFree(ctx->err);
        if (ctx->pos_slot_pool) (void)hipFree(ctx->pos_slot_pool);
        if (ctx->aux) (void)hipStreamDestroy(ctx->aux);
        for (auto& m : ctx->modules)
            if (m) (void)hipModuleUnload(m);
        delete ctx;
        return rc;
    };
    if ((e = hipSetDevice(device)) != hipSuccess) return bail(hip_fail(ctx, e, "hipSetDevice"));
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess)
        return bail(hip_fail(ctx, e, "hipGetDeviceProperties"));
    ctx->n_cu = prop.multiProcessorCount;
    std::snprintf(ctx->device_name, sizeof(ctx->device_name), "%s", prop.gcnArchName);
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        fprintf(stderr, "[tmac] device %d is %s; this library is built for gfx950 only\n", device,
                prop.gcnArchName);
        return bail(TMAC_ERR_UNSUPPORTED);
    }
    for (int i = 0; i < kCodeParts; i++)
        if ((e = hipModuleLoadData(&ctx->modules[i], tmac_attn_code_objects[i])) != hipSuccess)
            return bail(hip_fail(ctx, e, "hipModuleLoadData"));
    const char* mode_prefix[3] = {"tmac_decode_u", "tmac_decode_r", "tmac_layer"};
    for (int m = 0; m < 3; m++) {
        for (auto& sh : kShapes) {
            char name[64];
            std::snprintf(name, sizeof(name), "%s_g%d_kv%d", mode_prefix[m], sh[0], sh[1]);
            hipFunction_t f = nullptr;
            if ((e = get_function(ctx, &f, name)) != hipSuccess)
                return bail(hip_fail(ctx, e, name));
            ctx->decode[m][{sh[0], sh[1]}] = f;
            for (int dt = 0; dt < kNarrowTypes; dt++) {
                const char* tn = kTypeName[dt + 1];
                std::snprintf(name, sizeof(name), "%s_%s_g%d_kv%d", mode_prefix[m], tn, sh[0], sh[1]);
                if ((e = get_function(ctx, &f, name)) != hipSuccess)
                    return bail(hip_fail(ctx, e, name));
                ctx->decode_n[dt][m][{sh[0], sh[1]}] = f;
                std::snprintf(name, sizeof(name), "%s_%s_head8_g%d_kv%d", mode_prefix[m], tn, sh[0], sh[1]);
                if ((e = get_function(ctx, &f, name)) != hipSuccess)
                    return bail(hip_fail(ctx, e, name));
                ctx->head_n[dt][m][{sh[0], sh[1]}] = f;
            }
            for (int dt = 0; dt < kNarrowTypes; dt++) {  // MFMA decode (bf16, fp16, Q8_0)
                const char* mp[5] = {"tmac_mdecode_u", "tmac_mdecode_r", "tmac_mdecode_p", "tmac_mdecode_l",
                                     "tmac_mdecode_pl"};
                for (int mi = m; mi < 5; mi += 3) {  // m = 0, 1, 2 -> modes m and m + 3
                    std::snprintf(name, sizeof(name), "%s_%s_g%d_kv%d", mp[mi], kTypeName[dt + 1], sh[0], sh[1]);
                    if (get_function(ctx, &f, name) == hipSuccess) ctx->mdecode[dt][mi][{sh[0], sh[1]}] = f;
                }
                if (m < 2) {  // stream-K: m = 0 ragged, 1 paged
                    std::snprintf(name, sizeof(name), "tmac_mdecode_sk%s_%s_g%d_kv%d", m ? "_p" : "",
                                  kTypeName[dt + 1], sh[0], sh[1]);
                    if (get_function(ctx, &f, name) == hipSuccess) ctx->mdecode_sk[dt][m][{sh[0], sh[1]}] = f;
                }
            }
            if (m < 2) {  // paged kernels: m = kPagedDecode, kPagedLayer
                const char* pp = m == kPagedDecode ? "tmac_decode_p" : "tmac_layer_p";
                for (int dt = 0; dt < 4; dt++) {
                    std::snprintf(name, sizeof(name), "%s_%s_g%d_kv%d", pp, kTypeName[dt], sh[0], sh[1]);
                    if ((e = get_function(ctx, &f, name)) != hipSuccess)
                        return bail(hip_fail(ctx, e, name));
                    ctx->paged[dt][m][{sh[0], sh[1]}] = f;
                }
                if (m == kPagedDecode) {
                    std::snprintf(name, sizeof(name), "tmac_decode_sk_p_f32_g%d_kv%d", sh[0], sh[1]);
                    if ((e = get_function(ctx, &f, name)) != hipSuccess)
                        return bail(hip_fail(ctx, e, name));
                    ctx->decode_sk_p[{sh[0], sh[1]}] = f;
                } else {
                    std::snprintf(name, sizeof(name), "tmac_layer_sk_p_f32_g%d_kv%d", sh[0], sh[1]);
                    if ((e = get_function(ctx, &f, name)) != hipSuccess)
                        return bail(hip_fail(ctx, e, name));
                    ctx->layer_sk_p[{sh[0], sh[1]}] = f;
                    std::snprintf(name, sizeof(name), "tmac_layer_sk_combine_g%d_kv%d", sh[0], sh[1]);
                    if ((e = get_function(ctx, &f, name)) != hipSuccess)
                        return bail(hip_fail(ctx, e, name));
                    ctx->combine_sk_l[{sh[0], sh[1]}] = f;
                }
                std::snprintf(name, sizeof(name), "%s_combine_g%d_kv%d", pp, sh[0], sh[1]);
                if ((e = get_function(ctx, &f, name)) != hipSuccess)
                    return bail(hip_fail(ctx, e, name));
                ctx->combine_p[m][{sh[0], sh[1]}] = f;
            }
            std::snprintf(name, sizeof(name), "%s_g4w_g%d_kv%d", mode_prefix[m], sh[0], sh[1]);
            if ((e = get_function(ctx, &f, name)) != hipSuccess)
                return bail(hip_fail(ctx, e, name));
            ctx->decode4[m][{sh[0], sh[1]}] = f;
            std::snprintf(name, sizeof(name), "%s_head_g%d_kv%d", mode_prefix[m], sh[0], sh[1]);
            if ((e = get_function(ctx, &f, name)) != hipSuccess)
                return bail(hip_fail(ctx, e, name));
            ctx->head[m][{sh[0], sh[1]}] = f;
            std::snprintf(name, sizeof(name), "%s_head8_g%d_kv%d", mode_prefix[m], sh[0], sh[1]);
            if ((e = get_function(ctx, &f, name)) != hipSuccess)
                return bail(hip_fail(ctx, e, name));
            ctx->head8[m][{sh[0], sh[1]}] = f;
            std::snprintf(name, sizeof(name), "%s_head4_g%d_kv%d", mode_prefix[m], sh[0], sh[1]);
            if ((e = get_function(ctx, &f, name)) != hipSuccess)
                return bail(hip_fail(ctx, e, name));
            ctx->head4[m][{sh[0], sh[1]}] = f;
            for (int vs = 0; vs < 4; ++vs) {
                std::snprintf(name, sizeof(name), "%s_hv%d_g%d_kv%d", mode_prefix[m], 1 << vs, sh[0], sh[1]);
                if ((e = get_function(ctx, &f, name)) != hipSuccess)
                    return bail(hip_fail(ctx, e, name));
                ctx->hv[vs][m][{sh[0], sh[1]}] = f;
            }
            std::snprintf(name, sizeof(name), "%s_combine_g%d_kv%d", mode_prefix[m], sh[0], sh[1]);
            if ((e = get_function(ctx, &f, name)) != hipSuccess)
                return bail(hip_fail(ctx, e, name));
            ctx->combine[m][{sh[0], sh[1]}] = f;
            if (m == kModeRagged) {
                std::snprintf(name, sizeof(name), "tmac_decode_sk_g%d_kv%d", sh[0], sh[1]);
                if ((e = get_function(ctx, &f, name)) != hipSuccess)
                    return bail(hip_fail(ctx, e, name));
                ctx->decode_sk[{sh[0], sh[1]}] = f;
                std::snprintf(name, sizeof(name), "tmac_decode_sk_combine_g%d_kv%d", sh[0], sh[1]);
                if ((e = get_function(ctx, &f, name)) != hipSuccess)
                    return bail(hip_fail(ctx, e, name));
                ctx->combine_sk[{sh[0], sh[1]}] = f;
            }
            if (m == 0) {
                std::snprintf(name, sizeof(name), "tmac_prefill_g%d_kv%d", sh[0], sh[1]);
                if ((e = get_function(ctx, &f, name)) != hipSuccess)
                    return bail(hip_fail(ctx, e, name));
                ctx->prefill[{sh[0], sh[1]}] = f;
                static const char* const pack_type[4] = {"", "bf16_", "f16_", "q8_"};
                for (int pg = 0; pg < 2; ++pg)
                    for (int dt = 0; dt < 4; ++dt) {
                        if (ctx->prefill_pack[pg][dt].count(sh[1])) continue;
                        std::snprintf(name, sizeof(name), "tmac_prefill_pack_%s%skv%d", pg ? "p_" : "", pack_type[dt],
                                      sh[1]);
                        if ((e = get_function(ctx, &f, name)) != hipSuccess)
                            return bail(hip_fail(ctx, e, name));
                        ctx->prefill_pack[pg][dt][sh[1]] = f;
                    }
            }
        }
    }
    {
        const char* any_name[3] = {"tmac_decode_u_any", "tmac_decode_r_any", "tmac_layer_any"};
        for (int m = 0; m < 3; m++)
            if ((e = get_function(ctx, &ctx->any[m], any_name[m])) != hipSuccess)
                return bail(hip_fail(ctx, e, any_name[m]));
    }
    if ((e = get_function(ctx, &ctx->k_rope, "tmac_rope")) != hipSuccess ||
        (e = get_function(ctx, &ctx->k_copy, "tmac_copy")) != hipSuccess ||
        (e = get_function(ctx, &ctx->k_pos, "tmac_pos_update")) != hipSuccess ||
        (e = get_function(ctx, &ctx->k_qkv, "tmac_qkv")) != hipSuccess ||
        (e = get_function(ctx, &ctx->k_cvt16, "tmac_cvt16")) != hipSuccess ||
        (e = get_function(ctx, &ctx->k_kq, "tmac_matmul_kq")) != hipSuccess ||
        (e = get_function(ctx, &ctx->k_cvt_q8, "tmac_cvt_q8")) != hipSuccess)
        return bail(hip_fail(ctx, e, "hipModuleGetFunction"));
    if ((e = hipStreamCreateWithFlags(&ctx->aux, hipStreamNonBlocking)) != hipSuccess)
        return bail(hip_fail(ctx, e, "hipStreamCreateWithFlags"));
    if ((e = hipMalloc(&ctx->err, sizeof(int))) != hipSuccess) return bail(hip_fail(ctx, e, "hipMalloc"));
    if ((e = aux_fill(ctx, ctx->err, 0, sizeof(int))) != hipSuccess) return bail(hip_fail(ctx, e, "hipMemsetAsync"));
    if ((e = hipMalloc(&ctx->pos_slot_pool, (size_t)tmac::kPosSlotBlocks * tmac::kPosSlotBytes)) != hipSuccess)
        return bail(hip_fail(ctx, e, "hipMalloc"));
    if ((e = aux_fill(ctx, ctx->pos_slot_pool, 0xFF, (size_t)tmac::kPosSlotBlocks * tmac::kPosSlotBytes)) !=
        hipSuccess)
        return bail(hip_fail(ctx, e, "hipMemsetAsync"));  // every tag -1: no slot holds a row yet
    int rc = ensure_workspace(ctx, nullptr, (size_t)1 << 20);
    if (rc) return bail(rc);
    void* scratch = nullptr;
    if ((e = (hipError_t)tmac_scratch_setup(device, &scratch)) != hipSuccess)
        return bail(hip_fail(ctx, e, "hipGetSymbolAddress(scratch)"));
    ctx->scratch = static_cast<float*>(scratch);
    *out = ctx;
    return TMAC_OK;
}

int tmac_shutdown(tmac_context* ctx) {
    if (!ctx) return TMAC_ERR_NOT_INITIALIZED;
    if (ctx->modules[0]) {
        (void)hipSetDevice(ctx->device);
        // The caller has finished its work on this context; the device is
        // synchronized as well unless a step capture is in progress somewhere.
        (void)quiesce(ctx);
        if (ctx->aux) (void)hipStreamSynchronize(ctx->aux);
        for (auto& t : ctx->rope) (void)hipFree(t.dev);
        if (ctx->ws) (void)hipFree(ctx->ws);
        for (void* p : ctx->retired) (void)hipFree(p);
        for (tmac_graph* g : ctx->graphs) g->owner = nullptr;  // graphs destroyed later touch no context
        if (ctx->err) (void)hipFree(ctx->err);
        if (ctx->pos_slot_pool) (void)hipFree(ctx->pos_slot_pool);
        for (auto& m : ctx->modules)
            if (m) (void)hipModuleUnload(m);
    }
    if (ctx->aux) (void)hipStreamDestroy(ctx->aux);
    delete ctx;
    return TMAC_OK;
}

int tmac_attention_op(tmac_context* ctx, tmac_stream stream, const float* q, const float* k_cache,
                      const float* v_cache, float* out, int n_head, int n_kv_head, int head_dim,
                      int past_len) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!q || !k_cache || !v_cache || !out) return fail(ctx, TMAC_ERR_NULL_POINTER, "attention_op: null buffer");
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out))
        return fail(ctx, TMAC_ERR_MISALIGNED, "attention_op: buffers must be 16-byte aligned");
    Kernels kern;
    if ((rc = check_shape(ctx, n_head, n_kv_head, head_dim, &kern, kModeUniform))) return rc;
    if (past_len < 0 || past_len == INT_MAX) return fail(ctx, TMAC_ERR_INVALID_ARG, "past_len out of range");
    if ((rc = set_device(ctx))) return rc;
    DecodeArgs a{};
    a.q = q;
    a.k = k_cache;
    a.v = v_cache;
    a.out = out;
    a.seq_stride = 0;
    a.n_pos = past_len + 1;
    a.n_head = n_head;
    a.head_dim = head_dim;
    return run_decode(ctx, (hipStream_t)stream, kern, a, 1, past_len + 1, n_kv_head);
}

static int decode_batched_impl(tmac_context* ctx, tmac_stream stream, int dt, const float* q, const void* k,
                               const void* v, float* out, int n_seq, int n_head, int n_kv_head, int head_dim,
                               int n_pos, int64_t seq_stride) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!q || !k || !v || !out) return fail(ctx, TMAC_ERR_NULL_POINTER, "decode_batched: null buffer");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
        return fail(ctx, TMAC_ERR_MISALIGNED, "decode_batched: buffers must be 16-byte aligned");
    Kernels kern;
    if ((rc = check_shape(ctx, n_head, n_kv_head, head_dim, &kern, kModeUniform, dt))) return rc;
    if (n_seq < 0 || n_pos < 1 || seq_stride < 0 || (n_seq > 1 && seq_stride < n_pos))
        return fail(ctx, TMAC_ERR_INVALID_ARG, "decode_batched: need n_seq >= 0, n_pos >= 1, seq_stride >= n_pos");
    if (n_seq == 0) return TMAC_OK;
    if ((rc = set_device(ctx))) return rc;
    DecodeArgs a{};
    a.q = q;
    a.k = static_cast<const float*>(k);
    a.v = static_cast<const float*>(v);
    a.out = out;
    a.seq_stride = seq_stride;
    a.n_pos = n_pos;
    a.n_head = n_head;
    a.head_dim = head_dim;
    return run_decode(ctx, (hipStream_t)stream, kern, a, n_seq, n_pos, n_kv_head);
}

int tmac_attention_decode_batched(tmac_context* ctx, tmac_stream stream, const float* q, const float* k,
                                  const float* v, float* out, int n_seq, int n_head, int n_kv_head,
                                  int head_dim, int n_pos, int64_t seq_stride) {
    return decode_batched_impl(ctx, stream, TMAC_KV_F32, q, k, v, out, n_seq, n_head, n_kv_head, head_dim, n_pos,
                               seq_stride);
}

int tmac_attention_decode_batched_kv(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                                     const void* k, const void* v, float* out, int n_seq, int n_head,
                                     int n_kv_head, int head_dim, int n_pos, int64_t seq_stride) {
    return decode_batched_impl(ctx, stream, kv_dtype, q, k, v, out, n_seq, n_head, n_kv_head, head_dim, n_pos,
                               seq_stride);
}

static int decode_ragged_impl(tmac_context* ctx, tmac_stream stream, int dt, const float* q, const void* k_pool,
                              const void* v_pool, const int64_t* offsets, const int32_t* lengths, float* out,
                              int n_seq, int n_head, int n_kv_head, int head_dim, int max_len, int64_t total_rows) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!q || !k_pool || !v_pool || !offsets || !lengths || !out)
        return fail(ctx, TMAC_ERR_NULL_POINTER, "decode_ragged: null buffer");
    if (!aligned16(q) || !aligned16(k_pool) || !aligned16(v_pool) || !aligned16(out))
        return fail(ctx, TMAC_ERR_MISALIGNED, "decode_ragged: buffers must be 16-byte aligned");
    Kernels kern;
    if ((rc = check_shape(ctx, n_head, n_kv_head, head_dim, &kern, kModeRagged, dt))) return rc;
    if (n_seq < 0 || max_len < 1 || total_rows < 0)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "decode_ragged: need max_len >= 1, total_rows >= 0");
    if (n_seq == 0) return TMAC_OK;
    if ((rc = set_device(ctx))) return rc;
    DecodeArgs a{};
    a.q = q;
    a.k = static_cast<const float*>(k_pool);
    a.v = static_cast<const float*>(v_pool);
    a.out = out;
    a.offsets = offsets;
    a.lengths = lengths;
    a.n_head = n_head;
    a.head_dim = head_dim;
    unsigned threads = 0;
    if (!kern.any && ctx->opt_kernel != TMAC_KERNEL_HEAD && !use_head_kernel(ctx, n_seq, n_head, max_len)) {
        if (hipFunction_t sk = stream_k_kernel(ctx, dt, false, n_seq, n_head, n_kv_head, &threads))
            return run_decode_sk(ctx, (hipStream_t)stream, sk, threads,
                                 ctx->combine_sk.at({n_head / n_kv_head, n_kv_head}), a, n_seq, max_len);
    }
    return run_decode(ctx, (hipStream_t)stream, kern, a, n_seq, max_len, n_kv_head, total_rows);
}

int tmac_attention_decode_ragged(tmac_context* ctx, tmac_stream stream, const float* q,
                                 const float* k_pool, const float* v_pool, const int64_t* offsets,
                                 const int32_t* lengths, float* out, int n_seq, int n_head,
                                 int n_kv_head, int head_dim, int max_len, int64_t total_rows) {
    return decode_ragged_impl(ctx, stream, TMAC_KV_F32, q, k_pool, v_pool, offsets, lengths, out, n_seq, n_head,
                              n_kv_head, head_dim, max_len, total_rows);
}

int tmac_attention_decode_ragged_noalloc(tmac_context* ctx, tmac_stream stream, const float* q,
                                         const float* k_pool, const float* v_pool, const int64_t* offsets,
                                         const int32_t* lengths, float* out, int n_seq, int n_head,
                                         int n_kv_head, int head_dim, int max_len, int64_t total_rows) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!ctx->scratch) return fail(ctx, TMAC_ERR_NOT_INITIALIZED, "decode_ragged_noalloc: no scratch buffer");
    FixedWorkspace fixed(ctx, ctx->scratch, TMAC_SCRATCH_BYTES / sizeof(float));
    return decode_ragged_impl(ctx, stream, TMAC_KV_F32, q, k_pool, v_pool, offsets, lengths, out, n_seq, n_head,
                              n_kv_head, head_dim, max_len, total_rows);
}

int tmac_attention_decode_ragged_kv(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                                    const void* k_pool, const void* v_pool, const int64_t* offsets,
                                    const int32_t* lengths, float* out, int n_seq, int n_head, int n_kv_head,
                                    int head_dim, int max_len, int64_t total_rows) {
    return decode_ragged_impl(ctx, stream, kv_dtype, q, k_pool, v_pool, offsets, lengths, out, n_seq, n_head,
                              n_kv_head, head_dim, max_len, total_rows);
}

// The RoPE row cache of a device-side position counter (one block per
// counter, assigned on first use; null once the pool is used up).
static float2* pos_slots_for(tmac_context* ctx, const int* pos_dev) {
    auto it = ctx->pos_slot_of.find(pos_dev);
    if (it == ctx->pos_slot_of.end()) {
        if ((int)ctx->pos_slot_of.size() >= tmac::kPosSlotBlocks) return nullptr;
        it = ctx->pos_slot_of.emplace(pos_dev, (int)ctx->pos_slot_of.size()).first;
    }
    return reinterpret_cast<float2*>(ctx->pos_slot_pool + (size_t)it->second * tmac::kPosSlotBytes);
}

static int layer_common(tmac_context* ctx, hipStream_t stream, const float* q, const float* k_new,
                        const float* v_new, void* k_cache, void* v_cache, float* out, int n_head,
                        int n_kv_head, int head_dim, int pos, const int* pos_dev, int capacity,
                        float base, int dt = TMAC_KV_F32) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!q || !k_new || !v_new || !k_cache || !v_cache || !out)
        return fail(ctx, TMAC_ERR_NULL_POINTER, "layer_attention: null buffer");
    if (!aligned16(q) || !aligned16(k_new) || !aligned16(v_new) || !aligned16(k_cache) ||
        !aligned16(v_cache) || !aligned16(out))
        return fail(ctx, TMAC_ERR_MISALIGNED, "layer_attention: buffers must be 16-byte aligned");
    Kernels kern;
    if ((rc = check_shape(ctx, n_head, n_kv_head, head_dim, &kern, kModeLayer, dt))) return rc;
    if (capacity < 1) return fail(ctx, TMAC_ERR_INVALID_ARG, "layer_attention: capacity < 1");
    if (!pos_dev && (pos < 0 || pos >= capacity))
        return fail(ctx, TMAC_ERR_CAPACITY, "layer_attention: pos outside [0, capacity)");
    if (!(base > 0.f) || !std::isfinite(base)) return fail(ctx, TMAC_ERR_INVALID_ARG, "layer_attention: bad base");
    if ((rc = set_device(ctx))) return rc;
    const RopeTable* rt = nullptr;
    if ((rc = rope_table(ctx, stream, head_dim, base, pos_dev ? capacity : pos + 1, &rt))) return rc;
    DecodeArgs a{};
    a.q = q;
    a.k = static_cast<const float*>(k_cache);
    a.v = static_cast<const float*>(v_cache);
    a.out = out;
    a.n_head = n_head;
    a.k_new = k_new;
    a.v_new = v_new;
    a.k_out = static_cast<float*>(k_cache);
    a.v_out = static_cast<float*>(v_cache);
    a.rope_cs = rt->dev;
    a.rope_rows = rt->rows;
    a.pos_dev = pos_dev;
    // The row cache holds head_dim-64 rows (32 cos/sin pairs), which is what
    // tmac_pos_update copies and what the compiled kernels read.  The
    // any-shape kernel (any other head_dim) reads its table directly, and its
    // table is not recorded for the counter: a copy of 32 pairs from a table
    // of shorter rows would read past it.
    const bool row_cache = pos_dev && !kern.any && head_dim == kHeadDim;
    a.pos_slots = row_cache ? pos_slots_for(ctx, pos_dev) : nullptr;
    if (a.pos_slots) ctx->pos_table_of[pos_dev] = {rt->dev, rt->rows};
    a.pos_host = pos;
    a.capacity = capacity;
    a.head_dim = head_dim;
    return run_decode(ctx, stream, kern, a, 1, pos_dev ? capacity : pos + 1, n_kv_head);
}

int tmac_layer_attention(tmac_context* ctx, tmac_stream stream, const float* q, const float* k_new,
                         const float* v_new, float* k_cache, float* v_cache, float* out, int n_head,
                         int n_kv_head, int head_dim, int pos, int capacity, float base) {
    return layer_common(ctx, (hipStream_t)stream, q, k_new, v_new, k_cache, v_cache, out, n_head,
                        n_kv_head, head_dim, pos, nullptr, capacity, base);
}

int tmac_layer_attention_devpos(tmac_context* ctx, tmac_stream stream, const float* q,
                                const float* k_new, const float* v_new, float* k_cache,
                                float* v_cache, float* out, int n_head, int n_kv_head, int head_dim,
                                const int* pos_dev, int capacity, float base) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!pos_dev) return fail(ctx, TMAC_ERR_NULL_POINTER, "layer_attention_devpos: null pos_dev");
    return layer_common(ctx, (hipStream_t)stream, q, k_new, v_new, k_cache, v_cache, out, n_head,
                        n_kv_head, head_dim, 0, pos_dev, capacity, base);
}

int tmac_layer_attention_kv(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                            const float* k_new, const float* v_new, void* k_cache, void* v_cache, float* out,
                            int n_head, int n_kv_head, int head_dim, int pos, int capacity, float base) {
    return layer_common(ctx, (hipStream_t)stream, q, k_new, v_new, k_cache, v_cache, out, n_head, n_kv_head,
                        head_dim, pos, nullptr, capacity, base, kv_dtype);
}

int tmac_layer_attention_devpos_kv(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                                   const float* k_new, const float* v_new, void* k_cache, void* v_cache,
                                   float* out, int n_head, int n_kv_head, int head_dim, const int* pos_dev,
                                   int capacity, float base) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!pos_dev) return fail(ctx, TMAC_ERR_NULL_POINTER, "layer_attention_devpos: null pos_dev");
    return layer_common(ctx, (hipStream_t)stream, q, k_new, v_new, k_cache, v_cache, out, n_head, n_kv_head,
                        head_dim, 0, pos_dev, capacity, base, kv_dtype);
}

// Shared checks of the paged entry points.
static int check_paged(tmac_context* ctx, const char* what, const void* k_pages, const void* v_pages, int n_pages,
                       const int32_t* block_table, int max_pages, int max_len) {
    if (!k_pages || !v_pages || !block_table)
        return fail(ctx, TMAC_ERR_NULL_POINTER, std::string(what) + ": null buffer");
    if (!aligned16(k_pages) || !aligned16(v_pages) || (uintptr_t)block_table % 4)
        return fail(ctx, TMAC_ERR_MISALIGNED, std::string(what) + ": misaligned pool or block table");
    if (n_pages < 1 || max_pages < 1 || max_len < 1 || (int64_t)max_len > (int64_t)max_pages * kPageRows)
        return fail(ctx, TMAC_ERR_INVALID_ARG,
                    std::string(what) + ": need n_pages, max_pages >= 1 and 1 <= max_len <= 16 * max_pages");
    return TMAC_OK;
}

int tmac_attention_decode_paged(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                                const void* k_pages, const void* v_pages, int n_pages,
                                const int32_t* block_table, int max_pages, const int32_t* lengths,
                                float* out, int n_seq, int n_head, int n_kv_head, int head_dim,
                                int max_len, int64_t total_rows) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!q || !lengths || !out) return fail(ctx, TMAC_ERR_NULL_POINTER, "decode_paged: null buffer");
    if (!aligned16(q) || !aligned16(out) || (uintptr_t)lengths % 4)
        return fail(ctx, TMAC_ERR_MISALIGNED, "decode_paged: q and out must be 16-byte aligned");
    Kernels kern;
    if ((rc = check_shape(ctx, n_head, n_kv_head, head_dim, &kern, kModeRagged, kv_dtype, kPagedDecode))) return rc;
    if ((rc = check_paged(ctx, "decode_paged", k_pages, v_pages, n_pages, block_table, max_pages, max_len)))
        return rc;
    if (n_seq < 0 || total_rows < 0) return fail(ctx, TMAC_ERR_INVALID_ARG, "decode_paged: n_seq, total_rows >= 0");
    if (n_seq == 0) return TMAC_OK;
    if ((rc = set_device(ctx))) return rc;
    DecodeArgs a{};
    a.q = q;
    a.k = static_cast<const float*>(k_pages);
    a.v = static_cast<const float*>(v_pages);
    a.out = out;
    a.lengths = lengths;
    a.n_head = n_head;
    a.block_table = block_table;
    a.max_pages = max_pages;
    a.n_pages = n_pages;
    unsigned threads = 0;
    if (hipFunction_t sk = stream_k_kernel(ctx, kv_dtype, true, n_seq, n_head, n_kv_head, &threads))
        return run_decode_sk(ctx, (hipStream_t)stream, sk, threads, ctx->combine_sk.at({n_head / n_kv_head, n_kv_head}),
                             a, n_seq, max_len);
    return run_decode(ctx, (hipStream_t)stream, kern, a, n_seq, max_len, n_kv_head, total_rows);
}

int tmac_layer_attention_paged(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                               const float* k_new, const float* v_new, void* k_pages, void* v_pages,
                               int n_pages, const int32_t* block_table, int max_pages,
                               const int32_t* positions, float* out, int n_seq, int n_head, int n_kv_head,
                               int head_dim, int max_len, float base) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!q || !k_new || !v_new || !positions || !out)
        return fail(ctx, TMAC_ERR_NULL_POINTER, "layer_attention_paged: null buffer");
    if (!aligned16(q) || !aligned16(k_new) || !aligned16(v_new) || !aligned16(out) || (uintptr_t)positions % 4)
        return fail(ctx, TMAC_ERR_MISALIGNED, "layer_attention_paged: q, k_new, v_new, out must be 16-byte aligned");
    Kernels kern;
    if ((rc = check_shape(ctx, n_head, n_kv_head, head_dim, &kern, kModeLayer, kv_dtype, kPagedLayer))) return rc;
    if ((rc = check_paged(ctx, "layer_attention_paged", k_pages, v_pages, n_pages, block_table, max_pages,
                          max_len)))
        return rc;
    if (n_seq < 0) return fail(ctx, TMAC_ERR_INVALID_ARG, "layer_attention_paged: n_seq < 0");
    if (!(base > 0.f) || !std::isfinite(base))
        return fail(ctx, TMAC_ERR_INVALID_ARG, "layer_attention_paged: bad base");
    if (n_seq == 0) return TMAC_OK;
    if ((rc = set_device(ctx))) return rc;
    const RopeTable* rt = nullptr;
    if ((rc = rope_table(ctx, (hipStream_t)stream, head_dim, base, max_len, &rt))) return rc;
    DecodeArgs a{};
    a.q = q;
    a.k = static_cast<const float*>(k_pages);
    a.v = static_cast<const float*>(v_pages);
    a.out = out;
    a.n_head = n_head;
    a.k_new = k_new;
    a.v_new = v_new;
    a.k_out = static_cast<float*>(k_pages);
    a.v_out = static_cast<float*>(v_pages);
    a.rope_cs = rt->dev;
    a.rope_rows = rt->rows;
    a.capacity = (int)std::min<int64_t>((int64_t)max_pages * kPageRows, INT_MAX);
    a.positions = positions;
    a.block_table = block_table;
    a.max_pages = max_pages;
    a.n_pages = n_pages;
    if (kv_dtype == TMAC_KV_F32 && ctx->opt_split_len == 0 && use_stream_k(ctx, n_seq, kSkF32Layer)) {
        const std::pair<int, int> key{n_head / n_kv_head, n_kv_head};
        return run_decode_sk(ctx, (hipStream_t)stream, ctx->layer_sk_p.at(key), 256, ctx->combine_sk_l.at(key), a,
                             n_seq, max_len);
    }
    return run_decode(ctx, (hipStream_t)stream, kern, a, n_seq, max_len, n_kv_head);
}

int tmac_kv_convert(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* src, void* dst, int64_t n) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (kv_dtype != TMAC_KV_BF16 && kv_dtype != TMAC_KV_F16 && kv_dtype != TMAC_KV_Q8_0)
        return fail(ctx, TMAC_ERR_INVALID_ARG,
                    "kv_convert: kv_dtype must be TMAC_KV_BF16, TMAC_KV_F16 or TMAC_KV_Q8_0");
    if (!src || !dst) return fail(ctx, TMAC_ERR_NULL_POINTER, "kv_convert: null buffer");
    if (n < 0 || (n + 255) / 256 > INT_MAX) return fail(ctx, TMAC_ERR_INVALID_ARG, "kv_convert: bad count");
    const bool q8 = kv_dtype == TMAC_KV_Q8_0;
    if (q8 && n % kHeadDim) return fail(ctx, TMAC_ERR_INVALID_ARG, "kv_convert: Q8_0 needs n % 64 == 0");
    if (q8 ? (!aligned16(src) || (uintptr_t)dst % 4) : ((uintptr_t)src % 4 || (uintptr_t)dst % 2))
        return fail(ctx, TMAC_ERR_MISALIGNED, "kv_convert: misaligned");
    if (n == 0) return TMAC_OK;
    if ((rc = set_device(ctx))) return rc;
    CvtArgs a{src, dst, n, kv_dtype};
    if (q8)  // 32 head rows of 64 values per 256-thread workgroup
        return launch(ctx, ctx->k_cvt_q8, (unsigned)((n / kHeadDim + 31) / 32), 1, 256, (hipStream_t)stream, &a);
    return launch(ctx, ctx->k_cvt16, (unsigned)((n + 255) / 256), 1, 256, (hipStream_t)stream, &a);
}

// Chunked prefill over a contiguous cache (block_table null: sequence s at row
// s * seq_stride) or a paged one (n_pages pages, block_table [n_seq][max_pages]).
static int prefill_impl(tmac_context* ctx, tmac_stream stream, int dt, const float* q, const void* k_cache,
                        const void* v_cache, float* out, int n_seq, int n_q, int prefix_len, int64_t seq_stride,
                        int n_head, int n_kv_head, int head_dim, const int32_t* block_table = nullptr,
                        int max_pages = 0, int n_pages = 0) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (dt != TMAC_KV_F32 && dt != TMAC_KV_BF16 && dt != TMAC_KV_F16 && dt != TMAC_KV_Q8_0)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "prefill: kv_dtype must be TMAC_KV_F32, _BF16, _F16 or _Q8_0");
    if (!q || !k_cache || !v_cache || !out) return fail(ctx, TMAC_ERR_NULL_POINTER, "prefill: null buffer");
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out))
        return fail(ctx, TMAC_ERR_MISALIGNED, "prefill: buffers must be 16-byte aligned");
    if (head_dim != kHeadDim) return fail(ctx, TMAC_ERR_UNSUPPORTED, "prefill: head_dim must be 64");
    if ((rc = check_shape(ctx, n_head, n_kv_head, head_dim, nullptr, kModeUniform))) return rc;
    if (n_seq < 0 || n_q < 0 || prefix_len < 0 || (int64_t)prefix_len + n_q > INT_MAX)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "prefill: need n_seq, n_q, prefix_len >= 0");
    if (!block_table && n_seq > 1 && seq_stride < (int64_t)prefix_len + n_q)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "prefill: seq_stride must cover prefix_len + n_q rows");
    if (block_table && (n_pages < 1 || max_pages < 1 || (int64_t)prefix_len + n_q > (int64_t)max_pages * kPageRows))
        return fail(ctx, TMAC_ERR_INVALID_ARG, "prefill_paged: need n_pages, max_pages >= 1 and "
                                               "prefix_len + n_q <= 16 * max_pages");
    if ((int64_t)((n_q + kPrefillQueries - 1) / kPrefillQueries) * n_kv_head * n_seq > INT_MAX)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "prefill: too many (query block, kv head, sequence) units");
    if (n_seq == 0 || n_q == 0) return TMAC_OK;
    auto it = ctx->prefill.find({n_head / n_kv_head, n_kv_head});
    if (it == ctx->prefill.end()) return fail(ctx, TMAC_ERR_UNSUPPORTED, "prefill: unsupported group");
    if ((rc = set_device(ctx))) return rc;
    // bf16 tiles of rows 0 .. prefix_len + n_q - 1 per (sequence, kv head), in
    // the split-KV workspace, then the attention over them.
    const int n_qblk = (n_q + kPrefillQueries - 1) / kPrefillQueries;
    const int n_rows = prefix_len + n_q;
    const int n_tp = ((n_rows + kPrefillKeys - 1) / kPrefillKeys + kPrefillStageTiles - 1) / kPrefillStageTiles *
                     kPrefillStageTiles;
    const int64_t pack_blocks = (int64_t)n_tp * n_kv_head * n_seq;
    if (pack_blocks > INT_MAX) return fail(ctx, TMAC_ERR_INVALID_ARG, "prefill: too many cache tiles");
    const size_t pack_bytes = (size_t)pack_blocks * kPrefillTileElems * sizeof(uint16_t);
    if ((rc = ensure_workspace(ctx, (hipStream_t)stream, pack_bytes / sizeof(float)))) return rc;
    PrefillArgs a{q, static_cast<const float*>(k_cache), static_cast<const float*>(v_cache), out, seq_stride, n_q,
                  prefix_len, n_qblk, kQScale, reinterpret_cast<uint16_t*>(workspace(ctx)), n_tp, n_rows, 0, n_tp,
                  block_table, max_pages, n_pages, ctx->err, 0};
    if ((rc = launch(ctx, ctx->prefill_pack[block_table ? 1 : 0][dt].at(n_kv_head), (unsigned)pack_blocks, 1, 256,
                     (hipStream_t)stream, &a)))
        return rc;
    return launch(ctx, it->second, (unsigned)((int64_t)n_qblk * n_kv_head * n_seq), 1, kPrefillWaves * 64,
                  (hipStream_t)stream, &a);
}

int tmac_attention_prefill(tmac_context* ctx, tmac_stream stream, const float* q, const float* k_cache,
                           const float* v_cache, float* out, int n_seq, int n_q, int prefix_len,
                           int64_t seq_stride, int n_head, int n_kv_head, int head_dim) {
    return prefill_impl(ctx, stream, TMAC_KV_F32, q, k_cache, v_cache, out, n_seq, n_q, prefix_len, seq_stride,
                        n_head, n_kv_head, head_dim);
}

int tmac_attention_prefill_kv(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                              const void* k_cache, const void* v_cache, float* out, int n_seq, int n_q,
                              int prefix_len, int64_t seq_stride, int n_head, int n_kv_head, int head_dim) {
    return prefill_impl(ctx, stream, kv_dtype, q, k_cache, v_cache, out, n_seq, n_q, prefix_len, seq_stride,
                        n_head, n_kv_head, head_dim);
}

int tmac_attention_prefill_paged(tmac_context* ctx, tmac_stream stream, int kv_dtype, const float* q,
                                 const void* k_pages, const void* v_pages, int n_pages, const int32_t* block_table,
                                 int max_pages, float* out, int n_seq, int n_q, int prefix_len, int n_head,
                                 int n_kv_head, int head_dim) {
    if (!block_table) {
        const int rc = check_ctx(ctx);
        return rc ? rc : fail(ctx, TMAC_ERR_NULL_POINTER, "prefill_paged: null block table");
    }
    return prefill_impl(ctx, stream, kv_dtype, q, k_pages, v_pages, out, n_seq, n_q, prefix_len, 0, n_head,
                        n_kv_head, head_dim, block_table, max_pages, n_pages);
}

// Persistent tile copy for chunked prefill: tiles per (sequence, kv head) for
// `capacity` cache rows, as the attention kernel strides them.
static int prefill_tiles_per_head(int capacity) {
    return ((capacity + kPrefillKeys - 1) / kPrefillKeys + kPrefillStageTiles - 1) / kPrefillStageTiles *
           kPrefillStageTiles;
}

size_t tmac_prefill_tiles_bytes(int n_seq, int n_kv_head, int capacity) {
    if (n_seq < 0 || n_kv_head < 1 || capacity < 1) return 0;
    return (size_t)n_seq * (size_t)n_kv_head * (size_t)prefill_tiles_per_head(capacity) * kPrefillTileElems *
           sizeof(uint16_t);
}

int tmac_prefill_pack_rows(tmac_context* ctx, tmac_stream stream, int kv_dtype, const void* k_cache,
                           const void* v_cache, int64_t seq_stride, void* tiles, int capacity, int n_seq,
                           int n_kv_head, int head_dim, int row_begin, int row_end) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    const int dt = kv_dtype;
    if (dt != TMAC_KV_F32 && dt != TMAC_KV_BF16 && dt != TMAC_KV_F16 && dt != TMAC_KV_Q8_0)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "prefill_pack_rows: kv_dtype must be TMAC_KV_F32, _BF16, _F16 or _Q8_0");
    if (!k_cache || !v_cache || !tiles) return fail(ctx, TMAC_ERR_NULL_POINTER, "prefill_pack_rows: null buffer");
    if (!aligned16(k_cache) || !aligned16(v_cache) || !aligned16(tiles))
        return fail(ctx, TMAC_ERR_MISALIGNED, "prefill_pack_rows: buffers must be 16-byte aligned");
    if (head_dim != kHeadDim) return fail(ctx, TMAC_ERR_UNSUPPORTED, "prefill_pack_rows: head_dim must be 64");
    if (ctx->prefill_pack[0][dt].find(n_kv_head) == ctx->prefill_pack[0][dt].end())
        return fail(ctx, TMAC_ERR_UNSUPPORTED, "prefill_pack_rows: unsupported n_kv_head");
    if (n_seq < 0 || capacity < 1 || row_begin < 0 || row_end < row_begin || row_end > capacity)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "prefill_pack_rows: need 0 <= row_begin <= row_end <= capacity");
    if (n_seq > 1 && seq_stride < capacity)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "prefill_pack_rows: seq_stride must cover capacity rows");
    if (n_seq == 0 || row_end == row_begin) return TMAC_OK;
    const int n_tp = prefill_tiles_per_head(capacity);
    const int t0 = row_begin / kPrefillKeys, t1 = (row_end + kPrefillKeys - 1) / kPrefillKeys;
    const int64_t blocks = (int64_t)(t1 - t0) * n_kv_head * n_seq;
    if (blocks > INT_MAX || (int64_t)n_tp * n_kv_head * n_seq > INT_MAX)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "prefill_pack_rows: too many cache tiles");
    if ((rc = set_device(ctx))) return rc;
    // Tiles t0 .. t1 - 1, rows row_begin .. row_end - 1 from the cache; the
    // other rows of those tiles keep their contents.
    PrefillArgs a{nullptr, static_cast<const float*>(k_cache), static_cast<const float*>(v_cache), nullptr,
                  seq_stride, 0, 0, 0, kQScale, static_cast<uint16_t*>(tiles), n_tp, row_end, t0, t1 - t0,
                  nullptr, 0, 0, ctx->err, row_begin};
    return launch(ctx, ctx->prefill_pack[0][dt].at(n_kv_head), (unsigned)blocks, 1, 256, (hipStream_t)stream, &a);
}

int tmac_attention_prefill_tiles(tmac_context* ctx, tmac_stream stream, const float* q, const void* tiles,
                                 int capacity, float* out, int n_seq, int n_q, int prefix_len, int n_head,
                                 int n_kv_head, int head_dim) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!q || !tiles || !out) return fail(ctx, TMAC_ERR_NULL_POINTER, "prefill_tiles: null buffer");
    if (!aligned16(q) || !aligned16(tiles) || !aligned16(out))
        return fail(ctx, TMAC_ERR_MISALIGNED, "prefill_tiles: buffers must be 16-byte aligned");
    if (head_dim != kHeadDim) return fail(ctx, TMAC_ERR_UNSUPPORTED, "prefill_tiles: head_dim must be 64");
    if ((rc = check_shape(ctx, n_head, n_kv_head, head_dim, nullptr, kModeUniform))) return rc;
    if (n_seq < 0 || n_q < 0 || prefix_len < 0 || capacity < 1 || (int64_t)prefix_len + n_q > capacity)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "prefill_tiles: need n_seq, n_q, prefix_len >= 0 and "
                                               "prefix_len + n_q <= capacity");
    if ((int64_t)((n_q + kPrefillQueries - 1) / kPrefillQueries) * n_kv_head * n_seq > INT_MAX)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "prefill_tiles: too many (query block, kv head, sequence) units");
    if (n_seq == 0 || n_q == 0) return TMAC_OK;
    auto it = ctx->prefill.find({n_head / n_kv_head, n_kv_head});
    if (it == ctx->prefill.end()) return fail(ctx, TMAC_ERR_UNSUPPORTED, "prefill_tiles: unsupported group");
    if ((rc = set_device(ctx))) return rc;
    const int n_qblk = (n_q + kPrefillQueries - 1) / kPrefillQueries;
    PrefillArgs a{q, nullptr, nullptr, out, 0, n_q, prefix_len, n_qblk, kQScale,
                  static_cast<uint16_t*>(const_cast<void*>(tiles)), prefill_tiles_per_head(capacity),
                  prefix_len + n_q, 0, 0, nullptr, 0, 0, ctx->err, 0};
    return launch(ctx, it->second, (unsigned)((int64_t)n_qblk * n_kv_head * n_seq), 1, kPrefillWaves * 64,
                  (hipStream_t)stream, &a);
}

int tmac_pos_update(tmac_context* ctx, tmac_stream stream, int* pos_dev, int value, int add) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!pos_dev) return fail(ctx, TMAC_ERR_NULL_POINTER, "pos_update: null pointer");
    if ((rc = set_device(ctx))) return rc;
    PosArgs a{pos_dev, value, add ? 1 : 0, nullptr, nullptr, 0};
    // a counter the layer steps have used: also refresh its RoPE row cache
    const auto t = ctx->pos_table_of.find(pos_dev);
    const auto sl = ctx->pos_slot_of.find(pos_dev);
    if (t != ctx->pos_table_of.end() && sl != ctx->pos_slot_of.end()) {
        a.slots = reinterpret_cast<float2*>(ctx->pos_slot_pool + (size_t)sl->second * tmac::kPosSlotBytes);
        a.rope_cs = t->second.first;
        a.rope_rows = t->second.second;
    }
    return launch(ctx, ctx->k_pos, 1, 1, 64, (hipStream_t)stream, &a);
}

int tmac_rope_prepare(tmac_context* ctx, int head_dim, float base, int n_pos) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (head_dim < 2 || head_dim > kAnyMaxDim || head_dim % 2)
        return fail(ctx, TMAC_ERR_UNSUPPORTED, "rope: head_dim must be even, 2..256");
    if (n_pos < 1 || !(base > 0.f) || !std::isfinite(base))
        return fail(ctx, TMAC_ERR_INVALID_ARG, "rope_prepare: need n_pos >= 1 and base > 0");
    if ((rc = set_device(ctx))) return rc;
    const RopeTable* rt;
    return rope_table(ctx, nullptr, head_dim, base, n_pos, &rt);
}

int tmac_rope_op(tmac_context* ctx, tmac_stream stream, float* data, int n_heads, int head_dim, int pos,
                 float base) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!data) return fail(ctx, TMAC_ERR_NULL_POINTER, "rope_op: null data");
    if (!aligned16(data)) return fail(ctx, TMAC_ERR_MISALIGNED, "rope_op: data must be 16-byte aligned");
    if (head_dim < 2 || head_dim > kAnyMaxDim || head_dim % 2)
        return fail(ctx, TMAC_ERR_UNSUPPORTED, "rope_op: head_dim must be even, 2..256");
    if (n_heads < 0 || pos < 0 || pos == INT_MAX) return fail(ctx, TMAC_ERR_INVALID_ARG, "rope_op: bad n_heads/pos");
    if (!(base > 0.f) || !std::isfinite(base)) return fail(ctx, TMAC_ERR_INVALID_ARG, "rope_op: bad base");
    if (n_heads == 0) return TMAC_OK;
    if ((rc = set_device(ctx))) return rc;
    const RopeTable* rt = nullptr;
    if ((rc = rope_table(ctx, (hipStream_t)stream, head_dim, base, pos + 1, &rt))) return rc;
    RopeArgs a{data, rt->dev, nullptr, pos, n_heads, rt->rows, ctx->err, 1, 0, head_dim};
    const int threads = n_heads * (head_dim / 2);
    return launch(ctx, ctx->k_rope, (unsigned)((threads + 255) / 256), 1, 256, (hipStream_t)stream, &a);
}

int tmac_rope_rows(tmac_context* ctx, tmac_stream stream, float* data, int n_rows, int64_t row_stride, int n_heads,
                   int head_dim, int first_pos, float base) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!data) return fail(ctx, TMAC_ERR_NULL_POINTER, "rope_rows: null data");
    if (!aligned16(data) || row_stride % 4 != 0)
        return fail(ctx, TMAC_ERR_MISALIGNED, "rope_rows: data and rows must be 16-byte aligned");
    if (head_dim < 2 || head_dim > kAnyMaxDim || head_dim % 2)
        return fail(ctx, TMAC_ERR_UNSUPPORTED, "rope_rows: head_dim must be even, 2..256");
    if (n_rows < 0 || n_heads < 0 || first_pos < 0 || (int64_t)first_pos + n_rows > INT_MAX ||
        (n_rows > 1 && row_stride < (int64_t)n_heads * head_dim) ||
        (int64_t)n_rows * n_heads * (head_dim / 2) > INT_MAX)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "rope_rows: bad n_rows / row_stride / n_heads / first_pos");
    if (!(base > 0.f) || !std::isfinite(base)) return fail(ctx, TMAC_ERR_INVALID_ARG, "rope_rows: bad base");
    if (n_rows == 0 || n_heads == 0) return TMAC_OK;
    if ((rc = set_device(ctx))) return rc;
    const RopeTable* rt = nullptr;
    if ((rc = rope_table(ctx, (hipStream_t)stream, head_dim, base, first_pos + n_rows, &rt))) return rc;
    RopeArgs a{data, rt->dev, nullptr, first_pos, n_heads, rt->rows, ctx->err, n_rows, row_stride, head_dim};
    const int64_t threads = (int64_t)n_rows * n_heads * (head_dim / 2);
    return launch(ctx, ctx->k_rope, (unsigned)((threads + 255) / 256), 1, 256, (hipStream_t)stream, &a);
}

int tmac_elem_op(tmac_context* ctx, tmac_stream stream, int op, float* data, const float* aux, int dim) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (op != 0 && op != 2)
        return fail(ctx, TMAC_ERR_UNSUPPORTED,
                    "elem_op: op 0 (add: bias, residual) and op 2 (cache write) are supported; op 1 is the FFN");
    if (!data || !aux) return fail(ctx, TMAC_ERR_NULL_POINTER, "elem_op: null buffer");
    if (dim < 0) return fail(ctx, TMAC_ERR_INVALID_ARG, "elem_op: dim < 0");
    if (dim == 0) return TMAC_OK;
    if ((rc = set_device(ctx))) return rc;
    CopyArgs a{data, aux, dim, op == 0 ? 1 : 0};
    return launch(ctx, ctx->k_copy, (unsigned)((dim + 255) / 256), 1, 256, (hipStream_t)stream, &a);
}

static int qkv_common(tmac_context* ctx, hipStream_t stream, const void* w_q, const void* w_k, const void* w_v,
                      const float* x, const float* b_q, const float* b_k, const float* b_v, float* y_q,
                      float* y_k, float* y_v, int q_rows, int k_rows, int v_rows, int cols, int v_is_q8) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (q_rows < 0 || k_rows < 0 || v_rows < 0 || cols <= 0 || cols % 32)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "fused_qkv: rows >= 0 and cols a positive multiple of 32");
    const int64_t total = (int64_t)q_rows + k_rows + v_rows;
    if (total + kQkvWaves > INT_MAX || (int64_t)cols * 2 > INT_MAX)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "fused_qkv: too many rows");
    if (!x || (q_rows && (!w_q || !y_q)) || (k_rows && (!w_k || !y_k)) || (v_rows && (!w_v || !y_v)))
        return fail(ctx, TMAC_ERR_NULL_POINTER, "fused_qkv: null buffer");
    if (!aligned16(x) || ((uintptr_t)w_q | (uintptr_t)w_k | (uintptr_t)w_v) % 2 ||
        ((uintptr_t)y_q | (uintptr_t)y_k | (uintptr_t)y_v | (uintptr_t)b_q | (uintptr_t)b_k | (uintptr_t)b_v) % 4)
        return fail(ctx, TMAC_ERR_MISALIGNED,
                    "fused_qkv: x must be 16-byte aligned, weights 2-byte aligned, outputs and biases 4-byte");
    if (total == 0) return TMAC_OK;
    if ((rc = set_device(ctx))) return rc;
    QkvArgs a{{(const uint8_t*)w_q, (const uint8_t*)w_k, (const uint8_t*)w_v}, x, {b_q, b_k, b_v},
              {y_q, y_k, y_v}, {q_rows, k_rows, v_rows}, cols, v_is_q8 ? 1 : 0};
    return launch(ctx, ctx->k_qkv, (unsigned)((total + kQkvWaves - 1) / kQkvWaves), 1, kQkvWaves * 64, stream, &a);
}

int tmac_fused_qkv_op(tmac_context* ctx, tmac_stream stream, const void* w_q, const void* w_k, const void* w_v,
                      const float* x, float* y_q, float* y_k, float* y_v, int q_rows, int k_rows, int v_rows,
                      int cols, int v_is_q8) {
    return qkv_common(ctx, (hipStream_t)stream, w_q, w_k, w_v, x, nullptr, nullptr, nullptr, y_q, y_k, y_v, q_rows,
                      k_rows, v_rows, cols, v_is_q8);
}

int tmac_fused_qkv_bias(tmac_context* ctx, tmac_stream stream, const void* w_q, const void* w_k, const void* w_v,
                        const float* x, const float* b_q, const float* b_k, const float* b_v, float* y_q, float* y_k,
                        float* y_v, int q_rows, int k_rows, int v_rows, int cols, int v_is_q8) {
    return qkv_common(ctx, (hipStream_t)stream, w_q, w_k, w_v, x, b_q, b_k, b_v, y_q, y_k, y_v, q_rows, k_rows,
                      v_rows, cols, v_is_q8);
}

// A single weight matrix runs as the third segment of the projection kernel
// (rows of Q8_0 or Q5_0 blocks); the residual form passes y as its own bias.
static int matmul_common(tmac_context* ctx, hipStream_t stream, int qtype, int rows, int cols, const void* w,
                         const float* x, float* y, bool accumulate) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (qtype != TMAC_Q5_0 && qtype != TMAC_Q8_0 && qtype != TMAC_Q4_K && qtype != TMAC_Q6_K)
        return fail(ctx, TMAC_ERR_UNSUPPORTED, "matmul: weight type must be TMAC_Q5_0, _Q8_0, _Q4_K or _Q6_K");
    if (x && y && (const void*)x == (const void*)y)
        return fail(ctx, TMAC_ERR_INVALID_ARG, "matmul: x and y must not overlap");
    if (qtype == TMAC_Q4_K || qtype == TMAC_Q6_K) {
        if (rows < 0 || cols <= 0 || cols % 256 || rows > INT_MAX - kQkvWaves)
            return fail(ctx, TMAC_ERR_INVALID_ARG, "matmul: K-quant rows >= 0 and cols a positive multiple of 256");
        if (!w || !x || !y) return fail(ctx, TMAC_ERR_NULL_POINTER, "matmul: null buffer");
        if (!aligned16(x) || (uintptr_t)w % 2 || (uintptr_t)y % 4)
            return fail(ctx, TMAC_ERR_MISALIGNED, "matmul: x 16-byte, weights 2-byte, y 4-byte aligned");
        if (rows == 0) return TMAC_OK;
        if ((rc = set_device(ctx))) return rc;
        KqArgs a{(const uint8_t*)w, x, accumulate ? y : nullptr, y, rows, cols, qtype};
        return launch(ctx, ctx->k_kq, (unsigned)((rows + kQkvWaves - 1) / kQkvWaves), 1, kQkvWaves * 64, stream,
                      &a);
    }
    return qkv_common(ctx, stream, nullptr, nullptr, w, x, nullptr, nullptr, accumulate ? y : nullptr, nullptr,
                      nullptr, y, 0, 0, rows, cols, qtype == TMAC_Q8_0);
}

int tmac_matmul_q8_0(tmac_context* ctx, tmac_stream stream, int rows, int cols, const void* w, const float* x,
                     float* y) {
    return matmul_common(ctx, (hipStream_t)stream, TMAC_Q8_0, rows, cols, w, x, y, false);
}

int tmac_matmul_q5_0(tmac_context* ctx, tmac_stream stream, int rows, int cols, const void* w, const float* x,
                     float* y) {
    return matmul_common(ctx, (hipStream_t)stream, TMAC_Q5_0, rows, cols, w, x, y, false);
}

int tmac_matmul_q4_k(tmac_context* ctx, tmac_stream stream, int rows, int cols, const void* w, const float* x,
                     float* y) {
    return matmul_common(ctx, (hipStream_t)stream, TMAC_Q4_K, rows, cols, w, x, y, false);
}

int tmac_matmul_q6_k(tmac_context* ctx, tmac_stream stream, int rows, int cols, const void* w, const float* x,
                     float* y) {
    return matmul_common(ctx, (hipStream_t)stream, TMAC_Q6_K, rows, cols, w, x, y, false);
}

int tmac_matmul_add(tmac_context* ctx, tmac_stream stream, int qtype, int rows, int cols, const void* w,
                    const float* x, float* y) {
    return matmul_common(ctx, (hipStream_t)stream, qtype, rows, cols, w, x, y, true);
}

int tmac_set_option(tmac_context* ctx, int option, int64_t value) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (value < 0) return fail(ctx, TMAC_ERR_INVALID_ARG, "set_option: negative value");
    switch (option) {
        case TMAC_OPT_SPLIT_LEN: ctx->opt_split_len = value; return TMAC_OK;
        case TMAC_OPT_TARGET_GROUPS: ctx->opt_target_groups = value; return TMAC_OK;
        case TMAC_OPT_ROTATE:
            if (value > 1 << 20) return fail(ctx, TMAC_ERR_INVALID_ARG, "set_option: rotate too large");
            ctx->opt_rot_mul = value;
            return TMAC_OK;
        case TMAC_OPT_WAVE_ORDER:
            if (value > 1) return fail(ctx, TMAC_ERR_INVALID_ARG, "set_option: wave order is 0 or 1");
            ctx->opt_blocked = value;
            return TMAC_OK;
        case TMAC_OPT_GROUP_WAVES:
            if (value != 0 && value != 4 && value != 8)
                return fail(ctx, TMAC_ERR_INVALID_ARG, "set_option: group waves must be 0 (automatic), 4 or 8");
            ctx->opt_group_waves = value;
            return TMAC_OK;
        case TMAC_OPT_HEAD_WAVES:
            if (value != 4 && value != 8 && value != 16)
                return fail(ctx, TMAC_ERR_INVALID_ARG, "set_option: head waves must be 4, 8 or 16");
            ctx->opt_head_waves = value;
            return TMAC_OK;
        case TMAC_OPT_KERNEL:
            if (value < 0 || value > TMAC_KERNEL_HEADV)
                return fail(ctx, TMAC_ERR_INVALID_ARG, "set_option: bad kernel choice");
            ctx->opt_kernel = value;
            return TMAC_OK;
        case TMAC_OPT_HV_SPLIT:
            if (value != 1 && value != 2 && value != 4 && value != 8)
                return fail(ctx, TMAC_ERR_INVALID_ARG, "set_option: V split must be 1, 2, 4 or 8");
            ctx->opt_hv_split = value;
            return TMAC_OK;
        case TMAC_OPT_MFMA_DECODE:
            if (value > 1) return fail(ctx, TMAC_ERR_INVALID_ARG, "set_option: MFMA decode is 0 or 1");
            ctx->opt_mfma = value;
            return TMAC_OK;
        case TMAC_OPT_STREAM_K:
            if (value > 2) return fail(ctx, TMAC_ERR_INVALID_ARG, "set_option: stream-K is 0, 1 or 2");
            ctx->opt_stream_k = value;
            return TMAC_OK;
        default: return fail(ctx, TMAC_ERR_INVALID_ARG, "set_option: unknown option");
    }
}

int tmac_query_split(tmac_context* ctx, int n_seq, int n_pos, int n_head, int n_kv_head, int* split_len,
                     int* n_splits) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!split_len || !n_splits) return TMAC_ERR_NULL_POINTER;
    Kernels kern;
    if ((rc = check_shape(ctx, n_head, n_kv_head, kHeadDim, &kern, kModeUniform))) return rc;
    if (n_seq < 1 || n_pos < 1) return fail(ctx, TMAC_ERR_INVALID_ARG, "query_split: n_seq, n_pos >= 1");
    if (kern.any || use_head_kernel(ctx, n_seq, n_head, n_pos)) {
        *split_len = n_pos;
        *n_splits = 0;  // 0 = head kernel (one workgroup per query head)
        return TMAC_OK;
    }
    const int waves = ctx->opt_group_waves ? (int)ctx->opt_group_waves
                                           : auto_group_waves(ctx, n_seq, n_pos, n_kv_head, 0);
    choose_split(ctx, waves, n_seq, n_pos, n_kv_head, split_len, n_splits);
    return TMAC_OK;
}

int tmac_check_device_error(tmac_context* ctx) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if ((rc = set_device(ctx))) return rc;
    (void)quiesce(ctx);
    int v = 0;
    HIP_TRY(ctx, aux_copy(ctx, &v, ctx->err, sizeof(int), hipMemcpyDeviceToHost));
    if (v) {
        HIP_TRY(ctx, aux_fill(ctx, ctx->err, 0, sizeof(int)));
        return fail(ctx, TMAC_ERR_DEVICE_FAULT, "a kernel saw a device-side position outside its table or cache");
    }
    return TMAC_OK;
}

int tmac_step_begin(tmac_context* ctx, tmac_stream stream) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!stream) return fail(ctx, TMAC_ERR_INVALID_ARG, "step_begin: capture needs a created stream, not NULL");
    if ((rc = set_device(ctx))) return rc;
    HIP_TRY(ctx, hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal));
    g_captures.fetch_add(1);
    return TMAC_OK;
}

int tmac_step_end(tmac_context* ctx, tmac_stream stream, tmac_graph** graph) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!graph) return fail(ctx, TMAC_ERR_NULL_POINTER, "step_end: null graph handle");
    hipGraph_t g = nullptr;
    const bool was_capturing = capturing((hipStream_t)stream);
    const hipError_t ec = hipStreamEndCapture((hipStream_t)stream, &g);
    if (was_capturing) g_captures.fetch_sub(1);
    HIP_TRY(ctx, ec);
    if (*graph && (*graph)->exec) {
        hipGraphNode_t err_node = nullptr;
        hipGraphExecUpdateResult res;
        if (hipGraphExecUpdate((*graph)->exec, g, &err_node, &res) == hipSuccess &&
            res == hipGraphExecUpdateSuccess) {
            (void)hipGraphDestroy(g);
            return TMAC_OK;
        }
        (void)hipGetLastError();
        (void)hipGraphExecDestroy((*graph)->exec);
        (*graph)->exec = nullptr;
        forget_graph(*graph);
    }
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGraphInstantiate");
    if (!*graph) *graph = new tmac_graph();
    (*graph)->exec = exec;
    (*graph)->owner = ctx;
    ctx->live_graphs++;
    ctx->graphs.push_back(*graph);
    return TMAC_OK;
}

int tmac_graph_launch(tmac_context* ctx, tmac_graph* graph, tmac_stream stream) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!graph || !graph->exec) return fail(ctx, TMAC_ERR_NULL_POINTER, "graph_launch: empty graph");
    HIP_TRY(ctx, hipGraphLaunch(graph->exec, (hipStream_t)stream));
    return TMAC_OK;
}

int tmac_graph_destroy(tmac_context* ctx, tmac_graph* graph) {
    (void)ctx;
    if (!graph) return TMAC_OK;
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    tmac_context* owner = graph->owner;
    forget_graph(graph);
    delete graph;
    if (owner && owner->live_graphs == 0) free_retired(owner);
    return TMAC_OK;
}

int tmac_malloc(tmac_context* ctx, void** ptr, size_t bytes) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!ptr) return TMAC_ERR_NULL_POINTER;
    if ((rc = set_device(ctx))) return rc;
    HIP_TRY(ctx, hipMalloc(ptr, bytes ? bytes : 1));
    return TMAC_OK;
}

int tmac_free(tmac_context* ctx, void* ptr) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!ptr) return TMAC_OK;
    HIP_TRY(ctx, hipFree(ptr));
    return TMAC_OK;
}

static int copy_async(tmac_context* ctx, tmac_stream stream, void* dst, const void* src, size_t bytes,
                      hipMemcpyKind kind) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!bytes) return TMAC_OK;
    if (!dst || !src) return TMAC_ERR_NULL_POINTER;
    HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, kind, (hipStream_t)stream));
    return TMAC_OK;
}

int tmac_memcpy_h2d(tmac_context* ctx, tmac_stream s, void* d, const void* h, size_t n) {
    return copy_async(ctx, s, d, h, n, hipMemcpyHostToDevice);
}
int tmac_memcpy_d2h(tmac_context* ctx, tmac_stream s, void* h, const void* d, size_t n) {
    return copy_async(ctx, s, h, d, n, hipMemcpyDeviceToHost);
}
int tmac_memcpy_d2d(tmac_context* ctx, tmac_stream s, void* d, const void* src, size_t n) {
    return copy_async(ctx, s, d, src, n, hipMemcpyDeviceToDevice);
}

int tmac_memset(tmac_context* ctx, tmac_stream stream, void* dst, int value, size_t bytes) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!bytes) return TMAC_OK;
    if (!dst) return TMAC_ERR_NULL_POINTER;
    if (capturing((hipStream_t)stream))
        return fail(ctx, TMAC_ERR_CAPTURE,
                    "memset: the stream is capturing; a memset node does not reliably clear memory on graph "
                    "replays, so clear it before tmac_step_begin");
    HIP_TRY(ctx, hipMemsetAsync(dst, value, bytes, (hipStream_t)stream));
    return TMAC_OK;
}

int tmac_stream_create(tmac_context* ctx, tmac_stream* stream) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!stream) return TMAC_ERR_NULL_POINTER;
    if ((rc = set_device(ctx))) return rc;
    hipStream_t s;
    HIP_TRY(ctx, hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return TMAC_OK;
}

int tmac_stream_destroy(tmac_context* ctx, tmac_stream stream) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!stream) return TMAC_OK;
    HIP_TRY(ctx, hipStreamDestroy((hipStream_t)stream));
    return TMAC_OK;
}

int tmac_stream_synchronize(tmac_context* ctx, tmac_stream stream) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    HIP_TRY(ctx, hipStreamSynchronize((hipStream_t)stream));
    return TMAC_OK;
}

int tmac_device_synchronize(tmac_context* ctx) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if ((rc = set_device(ctx))) return rc;
    if (g_captures.load() != 0)
        return fail(ctx, TMAC_ERR_CAPTURE,
                    "device_synchronize: a step capture is in progress (a device-wide synchronize would end it); "
                    "synchronize the streams instead");
    HIP_TRY(ctx, hipDeviceSynchronize());
    return TMAC_OK;
}

int tmac_event_create(tmac_context* ctx, tmac_event* ev) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!ev) return TMAC_ERR_NULL_POINTER;
    hipEvent_t e;
    HIP_TRY(ctx, hipEventCreate(&e));
    *ev = e;
    return TMAC_OK;
}

int tmac_event_destroy(tmac_context* ctx, tmac_event ev) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (ev) HIP_TRY(ctx, hipEventDestroy((hipEvent_t)ev));
    return TMAC_OK;
}

int tmac_event_record(tmac_context* ctx, tmac_event ev, tmac_stream stream) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    HIP_TRY(ctx, hipEventRecord((hipEvent_t)ev, (hipStream_t)stream));
    return TMAC_OK;
}

int tmac_event_elapsed_ms(tmac_context* ctx, tmac_event start, tmac_event stop, float* ms) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!ms) return TMAC_ERR_NULL_POINTER;
    HIP_TRY(ctx, hipEventSynchronize((hipEvent_t)stop));
    HIP_TRY(ctx, hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return TMAC_OK;
}

int tmac_device_info(tmac_context* ctx, char* buf, size_t buf_len, int* n_cu) {
    int rc = check_ctx(ctx);
    if (rc) return rc;
    hipDeviceProp_t p;
    HIP_TRY(ctx, hipGetDeviceProperties(&p, ctx->device));
    if (n_cu) *n_cu = p.multiProcessorCount;
    if (buf && buf_len) {
        std::snprintf(buf, buf_len,
                      "{\"name\": \"%s\", \"arch\": \"%s\", \"cu\": %d, \"clock_khz\": %d, "
                      "\"mem_clock_khz\": %d, \"mem_bus_bits\": %d, \"hbm_bytes\": %zu, \"l2_bytes\": %d}",
                      p.name, p.gcnArchName, p.multiProcessorCount, p.clockRate, p.memoryClockRate,
                      p.memoryBusWidth, (size_t)p.totalGlobalMem, p.l2CacheSize);
    }
    return TMAC_OK;
}

// ---- TMAC weight file (load_tmac, tmac_gguf.cpp:1372-1425) ----

int tmac_model_load(tmac_context* ctx, const char* path, tmac_model** model) {
    if (ctx) {
        int rc = check_ctx(ctx);
        if (rc) return rc;
    }
    if (!path || !model) return fail(ctx, TMAC_ERR_NULL_POINTER, "model_load: null argument");
    *model = nullptr;
    std::unique_ptr<FILE, int (*)(FILE*)> f(std::fopen(path, "rb"), &std::fclose);
    if (!f) return fail(ctx, TMAC_ERR_IO, std::string("model_load: cannot open ") + path);
    if (fseeko(f.get(), 0, SEEK_END) != 0) return fail(ctx, TMAC_ERR_IO, "model_load: cannot seek");
    const uint64_t file_bytes = (uint64_t)ftello(f.get());
    fseeko(f.get(), 0, SEEK_SET);
    auto rd = [&](void* p, size_t n) { return std::fread(p, 1, n, f.get()) == n; };
    char magic[4];
    uint64_t n_tensors = 0;
    if (!rd(magic, 4) || std::memcmp(magic, "TMAC", 4) != 0 || !rd(&n_tensors, 8))
        return fail(ctx, TMAC_ERR_IO, "model_load: not a TMAC file");
    if (n_tensors > (file_bytes - 12) / 36)  // each entry holds at least 36 bytes of header
        return fail(ctx, TMAC_ERR_IO, "model_load: tensor count larger than the file");
    std::unique_ptr<tmac_model> m(new tmac_model());
    std::vector<uint64_t> file_off(n_tensors);
    size_t total = 0;
    for (uint64_t i = 0; i < n_tensors; i++) {
        tmac_model::Entry e;
        uint64_t name_len = 0;
        if (!rd(&name_len, 8) || name_len > file_bytes)
            return fail(ctx, TMAC_ERR_IO, "model_load: truncated at tensor " + std::to_string(i));
        const uint64_t keep = name_len < 128 ? name_len : 127;  // the reference keeps 127 characters
        e.name.resize(keep);
        if (!rd(&e.name[0], keep) || (name_len > keep && fseeko(f.get(), (off_t)(name_len - keep), SEEK_CUR) != 0))
            return fail(ctx, TMAC_ERR_IO, "model_load: truncated name at tensor " + std::to_string(i));
        e.name.resize(std::strlen(e.name.c_str()));  // a NUL inside the name ends it, as a C string read does
        if (!rd(&e.rows, 8) || !rd(&e.cols, 8) || !rd(&e.type, 4) || !rd(&e.n_bytes, 8))
            return fail(ctx, TMAC_ERR_IO, "model_load: truncated header at tensor " + std::to_string(i));
        const uint64_t at = (uint64_t)ftello(f.get());
        if (e.n_bytes > file_bytes - at)
            return fail(ctx, TMAC_ERR_IO, "model_load: data of tensor " + std::to_string(i) + " runs past the end");
        file_off[i] = at;
        fseeko(f.get(), (off_t)e.n_bytes, SEEK_CUR);
        total = (total + 255) & ~size_t(255);
        e.offset = total;
        total += e.n_bytes;
        m->index.emplace(e.name, m->tensors.size());  // keeps the first tensor of a name
        m->tensors.push_back(std::move(e));
    }
    m->bytes = total;
    std::vector<uint8_t> staging;
    if (ctx) {
        int rc = set_device(ctx);
        if (rc) return rc;
        if (total) HIP_TRY(ctx, hipMalloc(&m->blob, total));
        m->on_device = true;
    } else {
        m->host.reset(new uint8_t[total + 256]);  // aligned below, as device allocations are
        m->blob = reinterpret_cast<uint8_t*>((reinterpret_cast<uintptr_t>(m->host.get()) + 255) & ~uintptr_t(255));
    }
    for (size_t i = 0; i < m->tensors.size(); i++) {
        const tmac_model::Entry& e = m->tensors[i];
        uint8_t* dst = m->blob + e.offset;
        if (m->on_device) {
            staging.resize(e.n_bytes);
            dst = staging.data();
        }
        if (fseeko(f.get(), (off_t)file_off[i], SEEK_SET) != 0 || !rd(dst, e.n_bytes)) {
            if (m->on_device) (void)hipFree(m->blob);
            return fail(ctx, TMAC_ERR_IO, "model_load: cannot read tensor " + e.name);
        }
        if (m->on_device && e.n_bytes) {
            const hipError_t err = aux_copy(ctx, m->blob + e.offset, staging.data(), e.n_bytes,
                                            hipMemcpyHostToDevice);
            if (err != hipSuccess) {
                (void)hipFree(m->blob);
                return hip_fail(ctx, err, "model_load: hipMemcpyAsync");
            }
        }
    }
    *model = m.release();
    return TMAC_OK;
}

int tmac_model_count(const tmac_model* model) {
    return model ? (int)model->tensors.size() : -TMAC_ERR_NULL_POINTER;
}

static void fill_info(const tmac_model* m, size_t i, tmac_tensor_info* info) {
    const tmac_model::Entry& e = m->tensors[i];
    info->name = e.name.c_str();
    info->rows = e.rows;
    info->cols = e.cols;
    info->type = e.type;
    info->n_bytes = e.n_bytes;
    info->data = m->blob + e.offset;
}

int tmac_model_tensor(const tmac_model* model, int index, tmac_tensor_info* info) {
    if (!model || !info) return TMAC_ERR_NULL_POINTER;
    if (index < 0 || (size_t)index >= model->tensors.size()) return TMAC_ERR_INVALID_ARG;
    fill_info(model, (size_t)index, info);
    return TMAC_OK;
}

int tmac_model_find(const tmac_model* model, const char* name, tmac_tensor_info* info) {
    if (!model || !name || !info) return TMAC_ERR_NULL_POINTER;
    auto it = model->index.find(name);
    if (it == model->index.end()) return TMAC_ERR_NOT_FOUND;
    fill_info(model, it->second, info);
    return TMAC_OK;
}

int tmac_model_free(tmac_context* ctx, tmac_model* model) {
    if (!model) return TMAC_OK;
    if (model->on_device) {
        if (!ctx) return TMAC_ERR_INVALID_ARG;  // a device model needs its context
        int rc = set_device(ctx);
        if (rc) return rc;
        if (model->blob) (void)hipFree(model->blob);
    }
    delete model;
    return TMAC_OK;
}

}  // extern "C"
