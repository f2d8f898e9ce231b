// attn_kernels.hip -- gfx950 kernels for the reference's attention hot path:
// GQA decode attention over an fp32 KV cache (tmac_gguf.cpp:1093-1128), RoPE
// (tmac_gguf.cpp:990-1016) and the KV-cache row write (tmac_gguf.cpp:1090-1091).
//
// Built with `hipcc --genco --offload-arch=gfx950` into a code object that the
// host layer (tmac_attn.cpp) loads with hipModuleLoadData; every kernel is
// extern "C" and takes one argument struct from attn_args.h.
//
// Decode work decomposition (one workgroup = 4 waves = 256 lanes):
//   * grid = (split, sequence).  A split is a contiguous range of cache rows.
//   * A wave reads one "step" = 16 slots x 256 B of K and of V per iteration:
//     slot = (row within step, kv head); with 2 kv heads a step is 8 full
//     512-B cache rows, i.e. 4 KB of K and 4 KB of V, read with 16-byte loads.
//   * Each slot is served by 4 lanes; lane c of a slot owns the 16 dims
//     {16i + 4c + j : i, j in 0..3}, so one 16-byte load instruction covers a
//     64-byte run of every row it touches.
//   * Every lane keeps the (pre-scaled) query of all G heads of its kv group
//     in registers: the K/V row it loads is used by all G = n_head/n_kv_head
//     query heads of that group without being re-read (GQA sharing).
//   * q.k partial sums over a lane's 16 dims are reduced across the 4 lanes of
//     the slot with two DPP quad_perm adds; all 4 lanes end with the same score.
//   * Softmax is online, in base 2, with one running max per (wave, head)
//     shared by all slots of the wave.  The max is only raised when a score
//     exceeds it by more than kTau (a wave-uniform, rare branch), so the
//     common step has no cross-lane traffic besides the two DPP adds.
//   * End of wave: slots are summed with xor-shuffles (same max, no rescale);
//     waves are merged in LDS with a log-sum-exp rescale; splits of one
//     sequence are merged by the last workgroup to arrive (device-scope
//     fence + atomic counter that the merging workgroup resets to zero).
#include <hip/hip_runtime.h>

#include "attn_args.h"

using namespace tmac;

namespace {

constexpr float kTau = 8.0f;  // lazy-rescale threshold (log2 units): weights stay <= 2^8
constexpr float kNegInf = -__builtin_inff();

enum Mode { kUniform = 0, kRagged = 1, kLayer = 2 };

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Rotation of one adjacent pair, exactly as tmac_gguf.cpp:999-1001 rounds it:
// each product rounded, then the sum/difference rounded (no fused multiply-add).
__device__ __forceinline__ void rotate_pair(float& x0, float& x1, float c, float s) {
#pragma clang fp contract(off)
    const float a = x0 * c;
    const float b = x1 * s;
    const float e = x0 * s;
    const float f = x1 * c;
    x0 = a - b;
    x1 = e + f;
}

// Applies RoPE to a lane's 16 dims {16i + 4c + j} of one head.  Pairs (d, d+1)
// with d even never straddle a lane: dims 4m..4m+3 hold pairs 2m and 2m+1.
__device__ __forceinline__ void rope16(float (&x)[16], const float2* __restrict__ cs_row, int c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 t = *reinterpret_cast<const float4*>(cs_row + 8 * i + 2 * c);
        rotate_pair(x[4 * i + 0], x[4 * i + 1], t.x, t.y);
        rotate_pair(x[4 * i + 2], x[4 * i + 3], t.z, t.w);
    }
}

__device__ __forceinline__ void load16(float (&x)[16], const float* __restrict__ p) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 t = *reinterpret_cast<const float4*>(p + 16 * i);
        x[4 * i + 0] = t.x;
        x[4 * i + 1] = t.y;
        x[4 * i + 2] = t.z;
        x[4 * i + 3] = t.w;
    }
}

__device__ __forceinline__ void store16(float* __restrict__ p, const float (&x)[16]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
        *reinterpret_cast<float4*>(p + 16 * i) =
            make_float4(x[4 * i + 0], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
}

template <int G>
struct State {
    float m[G];       // running max (log2 domain), identical in every lane of a kv group
    float l[G];       // running sum of weights
    float acc[G][16]; // running sum of weight * v over this lane's 16 dims
};

template <int G>
__device__ __forceinline__ void state_init(State<G>& st) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
        st.m[g] = kNegInf;
        st.l[g] = 0.f;
#pragma unroll
        for (int t = 0; t < 16; ++t) st.acc[g][t] = 0.f;
    }
}

// One step: this lane's slot sees one cache row (kf/vf = its 16 dims of the
// row's kv head) or nothing (valid == false, only when MASKED).
template <int G, int KV, bool MASKED>
__device__ __forceinline__ void attend(const float (&q)[G][16], State<G>& st, const float (&kf)[16],
                                       const float (&vf)[16], bool valid) {
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float a = q[g][0] * kf[0];
#pragma unroll
        for (int t = 1; t < 16; ++t) a = fmaf(q[g][t], kf[t], a);
        s[g] = a;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        s[g] += dpp<0xB1>(s[g]);  // quad_perm [1,0,3,2]
        s[g] += dpp<0x4E>(s[g]);  // quad_perm [2,3,0,1]
        if (MASKED) s[g] = valid ? s[g] : kNegInf;
    }
    bool need = false;
#pragma unroll
    for (int g = 0; g < G; ++g) need |= (s[g] - st.m[g]) > kTau;
    if (__any(need)) {
        // Raise the shared max to the step's max (rare after the first step).
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float mx = s[g];
#pragma unroll
            for (int mask = 4 * KV; mask < 64; mask <<= 1) mx = fmaxf(mx, __shfl_xor(mx, mask));
            const float mn = fmaxf(st.m[g], mx);
            const float alpha = (st.m[g] == kNegInf) ? 0.f : fast_exp2(st.m[g] - mn);
            st.l[g] *= alpha;
#pragma unroll
            for (int t = 0; t < 16; ++t) st.acc[g][t] *= alpha;
            st.m[g] = mn;
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float e = fast_exp2(s[g] - st.m[g]);  // 0 for masked slots (s = -inf)
        st.l[g] += e;
#pragma unroll
        for (int t = 0; t < 16; ++t) st.acc[g][t] = fmaf(e, vf[t], st.acc[g][t]);
    }
}

// Attends this wave's share of `n_rows` cache rows starting at kb/vb.  Steps
// are dealt round-robin to the NW waves of the workgroup, so the workgroup
// streams its range front to back.  One step of K/V is prefetched ahead.
template <int G, int KV, int NW>
__device__ __forceinline__ void attend_rows(const float* __restrict__ kb, const float* __restrict__ vb,
                                            int n_rows, int wave, int lane_off, int lane_row,
                                            int lane_col, const float (&q)[G][16], State<G>& st) {
    constexpr int PPS = 16 / KV;       // rows per step
    constexpr int ROW = KV * kHeadDim; // floats per cache row
    constexpr int STEP = PPS * ROW;    // floats per step (= 1024)
    const int full = n_rows / PPS;     // steps whose rows are all in range
    int t = wave;
    if (t * PPS >= n_rows) return;

    float ka[16], va[16], kb2[16], vb2[16];
    auto load = [&](int step, float (&kk)[16], float (&vv)[16]) {
        if (step < full) {
            const int off = step * STEP + lane_off;
            load16(kk, kb + off);
            load16(vv, vb + off);
        } else {
            const int r = min(step * PPS + lane_row, n_rows - 1);
            const int off = r * ROW + lane_col;
            load16(kk, kb + off);
            load16(vv, vb + off);
        }
    };
    auto compute = [&](int step, const float (&kk)[16], const float (&vv)[16]) {
        if (step < full)
            attend<G, KV, false>(q, st, kk, vv, true);
        else
            attend<G, KV, true>(q, st, kk, vv, step * PPS + lane_row < n_rows);
    };

    load(t, ka, va);
    while (true) {
        int tn = t + NW;
        bool more = tn * PPS < n_rows;
        if (more) load(tn, kb2, vb2);
        compute(t, ka, va);
        if (!more) break;
        t = tn;
        tn = t + NW;
        more = tn * PPS < n_rows;
        if (more) load(tn, ka, va);
        compute(t, kb2, vb2);
        if (!more) break;
        t = tn;
    }
}

// Merges one workgroup's NW wave states; writes either the final output
// (single split) or this split's partial, then merges splits in the last
// workgroup to arrive.
template <int G, int KV, int NW>
__device__ __forceinline__ void finish(State<G>& st, int lane, int wave, int n_head, int split,
                                       int n_act, float* __restrict__ out_seq,
                                       float* __restrict__ ws_seq, int* __restrict__ counter) {
    // 1. Sum the slots of each kv group inside the wave (they share the max).
#pragma unroll
    for (int mask = 4 * KV; mask < 64; mask <<= 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            st.l[g] += __shfl_xor(st.l[g], mask);
#pragma unroll
            for (int t = 0; t < 16; ++t) st.acc[g][t] += __shfl_xor(st.acc[g][t], mask);
        }
    }
    // 2. Waves -> LDS.
    __shared__ float s_acc[NW][KV * G][kHeadDim];
    __shared__ float s_m[NW][KV * G];
    __shared__ float s_l[NW][KV * G];
    __shared__ int s_last;
    const int slot = lane >> 2, c = lane & 3;
    if (slot < KV) {  // row 0 of the step holds the wave total for kv head `slot`
        const int kv = slot;
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) s_acc[wave][kv * G + g][16 * i + 4 * c + j] = st.acc[g][4 * i + j];
            if (c == 0) {
                s_m[wave][kv * G + g] = st.m[g];
                s_l[wave][kv * G + g] = st.l[g];
            }
        }
    }
    __syncthreads();
    // 3. Merge waves: thread per (head, dim).
    const bool direct = (n_act == 1);
    for (int idx = threadIdx.x; idx < KV * G * kHeadDim; idx += NW * 64) {
        const int h = idx >> 6, d = idx & 63;
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][h]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float mw = s_m[w][h];
            const float sc = (mw == kNegInf) ? 0.f : fast_exp2(mw - M);
            L = fmaf(s_l[w][h], sc, L);
            A = fmaf(s_acc[w][h][d], sc, A);
        }
        if (direct) {
            out_seq[idx] = A / L;
        } else {
            float* p = ws_seq + ((size_t)split * n_head + h) * kPartialStride;
            p[d] = A;
            if (d == 0) {
                p[kHeadDim] = M;
                p[kHeadDim + 1] = L;
            }
        }
    }
    if (direct) return;
    // 4. Publish this split; the last workgroup of the sequence merges all.
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int prev = atomicAdd(counter, 1);
        s_last = (prev == n_act - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int idx = threadIdx.x; idx < n_head * kHeadDim; idx += NW * 64) {
        const int h = idx >> 6, d = idx & 63;
        float M = kNegInf;
        for (int sp = 0; sp < n_act; ++sp) M = fmaxf(M, ws_seq[((size_t)sp * n_head + h) * kPartialStride + kHeadDim]);
        float L = 0.f, A = 0.f;
        for (int sp = 0; sp < n_act; ++sp) {
            const float* p = ws_seq + ((size_t)sp * n_head + h) * kPartialStride;
            const float mw = p[kHeadDim];
            const float sc = (mw == kNegInf) ? 0.f : fast_exp2(mw - M);
            L = fmaf(p[kHeadDim + 1], sc, L);
            A = fmaf(p[d], sc, A);
        }
        out_seq[idx] = A / L;
    }
    if (threadIdx.x == 0) *counter = 0;  // ready for the next launch
}

template <int G, int KV, int NW, int MODE>
__device__ __forceinline__ void decode_body(const DecodeArgs& a) {
    constexpr int ROW = KV * kHeadDim;
    constexpr int NH = KV * G;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int split = blockIdx.x;
    const int seq = blockIdx.y;

    const float* kseq;
    const float* vseq;
    int n_pos, mem_rows, pos = 0;
    if (MODE == kUniform) {
        n_pos = a.n_pos;
        const size_t base = (size_t)seq * (size_t)a.seq_stride * ROW;
        kseq = a.k + base;
        vseq = a.v + base;
        mem_rows = n_pos;
    } else if (MODE == kRagged) {
        n_pos = a.lengths[seq];
        const size_t base = (size_t)a.offsets[seq] * ROW;
        kseq = a.k + base;
        vseq = a.v + base;
        mem_rows = n_pos;
    } else {
        pos = a.pos_dev ? *a.pos_dev : a.pos_host;
        if (pos < 0 || pos >= a.capacity || pos >= a.rope_rows) {
            if (split == 0 && threadIdx.x == 0) atomicOr(a.err, 1);
            return;
        }
        n_pos = pos + 1;
        kseq = a.k;
        vseq = a.v;
        mem_rows = pos;  // row `pos` is the new token, attended from registers
    }
    float* out_seq = a.out + (size_t)seq * NH * kHeadDim;
    if (n_pos <= 0) {  // ragged sequence with no rows: defined as a zero output
        if (split == 0)
            for (int i = threadIdx.x; i < NH * kHeadDim; i += NW * 64) out_seq[i] = 0.f;
        return;
    }
    const int n_act = (n_pos + a.split_len - 1) / a.split_len;
    if (n_act > a.n_splits) {  // ragged length above the max_len the grid was sized for
        if (split == 0) {
            for (int i = threadIdx.x; i < NH * kHeadDim; i += NW * 64) out_seq[i] = __builtin_nanf("");
            if (threadIdx.x == 0) atomicOr(a.err, 2);
        }
        return;
    }
    if (split >= n_act) return;
    const int r0 = split * a.split_len;
    const int r1 = min(r0 + a.split_len, mem_rows);

    const int slot = lane >> 2, c = lane & 3;
    const int kv = slot % KV, lane_row = slot / KV;
    const int lane_col = kv * kHeadDim + 4 * c;
    const int lane_off = lane_row * ROW + lane_col;

    // Query of the G heads of this lane's kv group, this lane's 16 dims.
    float q[G][16];
    const float* qg = a.q + ((size_t)seq * NH + kv * G) * kHeadDim + 4 * c;
    const float2* cs_row = nullptr;
    if (MODE == kLayer) cs_row = a.rope_cs + (size_t)pos * (kHeadDim / 2);
#pragma unroll
    for (int g = 0; g < G; ++g) {
        load16(q[g], qg + g * kHeadDim);
        if (MODE == kLayer) rope16(q[g], cs_row, c);
#pragma unroll
        for (int t = 0; t < 16; ++t) q[g][t] *= a.qscale;
    }

    State<G> st;
    state_init(st);
    attend_rows<G, KV, NW>(kseq + (size_t)r0 * ROW, vseq + (size_t)r0 * ROW, max(r1 - r0, 0), wave,
                           lane_off, lane_row, lane_col, q, st);

    if (MODE == kLayer && split == n_act - 1 && wave == 0) {
        // The new token (row `pos`): RoPE its k, write k/v to the cache row
        // (tmac_gguf.cpp:1090-1091) and attend it from registers.
        const bool mine = (lane_row == 0);
        float kf[16], vf[16];
        if (mine) {
            load16(kf, a.k_new + lane_col);
            load16(vf, a.v_new + lane_col);
            rope16(kf, cs_row, c);
            store16(const_cast<float*>(a.k) + (size_t)pos * ROW + lane_col, kf);
            store16(const_cast<float*>(a.v) + (size_t)pos * ROW + lane_col, vf);
        } else {
#pragma unroll
            for (int t = 0; t < 16; ++t) kf[t] = vf[t] = 0.f;
        }
        attend<G, KV, true>(q, st, kf, vf, mine);
    }

    float* ws_seq = a.ws ? a.ws + (size_t)seq * a.n_splits * NH * kPartialStride : nullptr;
    finish<G, KV, NW>(st, lane, wave, NH, split, n_act, out_seq, ws_seq, a.counters ? a.counters + seq : nullptr);
}

}  // namespace

#define TMAC_DECODE_KERNELS(G, KV)                                                          \
    extern "C" __global__ __launch_bounds__(kWavesPerGroup * 64) void tmac_decode_u_g##G##_kv##KV( \
        DecodeArgs a) {                                                                     \
        decode_body<G, KV, kWavesPerGroup, kUniform>(a);                                    \
    }                                                                                       \
    extern "C" __global__ __launch_bounds__(kWavesPerGroup * 64) void tmac_decode_r_g##G##_kv##KV( \
        DecodeArgs a) {                                                                     \
        decode_body<G, KV, kWavesPerGroup, kRagged>(a);                                     \
    }                                                                                       \
    extern "C" __global__ __launch_bounds__(kWavesPerGroup * 64) void tmac_layer_g##G##_kv##KV(    \
        DecodeArgs a) {                                                                     \
        decode_body<G, KV, kWavesPerGroup, kLayer>(a);                                      \
    }

// (query heads per kv head, kv heads).  Qwen2-0.5B is (7, 2).
TMAC_DECODE_KERNELS(7, 2)
TMAC_DECODE_KERNELS(1, 1)
TMAC_DECODE_KERNELS(1, 2)
TMAC_DECODE_KERNELS(2, 2)
TMAC_DECODE_KERNELS(4, 2)
TMAC_DECODE_KERNELS(4, 4)
TMAC_DECODE_KERNELS(8, 1)

// RoPE in place, one lane per (head, pair): tmac_gguf.cpp:992-1003 for one
// tensor, i.e. what rope_op (metal_backend.hpp:381) dispatches.
extern "C" __global__ __launch_bounds__(256) void tmac_rope(RopeArgs a) {
    const int pos = a.pos_dev ? *a.pos_dev : a.pos_host;
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (pos < 0 || pos >= a.rope_rows) {
        if (gid == 0) atomicOr(a.err, 1);
        return;
    }
    const int head = gid >> 5, pair = gid & 31;
    if (head >= a.n_heads) return;
    const float2 t = a.rope_cs[(size_t)pos * (kHeadDim / 2) + pair];
    float2* p = reinterpret_cast<float2*>(a.x + head * kHeadDim) + pair;
    float2 x = *p;
    rotate_pair(x.x, x.y, t.x, t.y);
    *p = x;
}

// dst[i] = src[i]: the cache-row write of elem_op(2, ...) (kernel_elem op 2).
extern "C" __global__ __launch_bounds__(256) void tmac_copy(CopyArgs a) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < a.n) a.dst[i] = a.src[i];
}

// Device-side position for graph replays: *pos = value, or *pos += value.
extern "C" __global__ __launch_bounds__(64) void tmac_pos_update(PosArgs a) {
    if (threadIdx.x == 0) *a.pos = a.add ? *a.pos + a.value : a.value;
}
