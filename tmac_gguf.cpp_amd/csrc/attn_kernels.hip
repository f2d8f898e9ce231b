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
//   * A wave reads one "step" per iteration: 8 slots x 256 B of K and of V,
//     slot = (row within the step, kv head).  With 2 kv heads a step is 4 full
//     512-B cache rows (2 KB of K, 2 KB of V), read with 16-byte loads.
//   * Each slot is served by 8 lanes; lane c owns the dims {4c..4c+3} and
//     {32+4c..32+4c+3}, so each 16-byte load instruction covers whole 128-byte
//     runs of the rows it touches.
//   * Every lane keeps the pre-scaled query of all G heads of its kv group in
//     registers: the K/V row it loads serves all G = n_head/n_kv_head query
//     heads of the group without being re-read (GQA sharing).
//   * q.k partial sums are reduced over the 8 lanes of a slot with three DPP
//     adds (quad_perm x2, row_half_mirror); all 8 lanes end with the same score.
//   * Softmax is online, in base 2, with one running max per (wave, head)
//     shared by all slots of the wave.  The max is raised only when a score
//     exceeds it by more than kTau (a wave-uniform, rare branch), so a common
//     step has no cross-lane traffic besides the three DPP adds.
//   * K/V of the next DEPTH-1 steps are in flight while a step is computed.
//   * End of wave: slots are summed with xor-shuffles (same max, no rescale);
//     waves are merged in LDS with a log-sum-exp rescale.  With one split the
//     workgroup writes the output; otherwise it writes its (m, l, acc) partial
//     and tmac_combine_* merges the splits in a second, stream-ordered launch
//     (no device-scope fences or counters inside the decode kernel).
#include <hip/hip_runtime.h>

#include "attn_args.h"

// The kernels are instantiated in four parts, each built into its own code
// object (in parallel): 0 the fp32 decode family, 1 the bf16 / fp16 / Q8_0
// VALU decode family, 2 the paged family, 3 the MFMA decode, prefill,
// projection and small kernels.  Without TMAC_PART every kernel is built.
#ifndef TMAC_PART
#define TMAC_PART -1
#endif
#define TMAC_IN_PART(p) (TMAC_PART < 0 || TMAC_PART == (p))

using namespace tmac;

namespace {

constexpr float kTau = 8.0f;  // lazy-rescale threshold (log2 units): weights stay <= 2^8
constexpr float kNegInf = -__builtin_inff();
constexpr int kLanesPerSlot = 8;
constexpr int kDimsPerLane = kHeadDim / kLanesPerSlot;  // 8
constexpr int kSlots = 64 / kLanesPerSlot;              // 8 (row, kv) slots per wave step

enum Mode { kUniform = 0, kRagged = 1, kLayer = 2, kPaged = 3, kPagedLayer = 4 };
constexpr bool is_layer(int m) { return m == kLayer || m == kPagedLayer; }
constexpr bool is_paged(int m) { return m == kPaged || m == kPagedLayer; }

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over the 8 lanes of a slot; every lane receives the same bits.
__device__ __forceinline__ float slot_sum(float x) {
    x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
    x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
    x += dpp<0x141>(x);  // row_half_mirror: lane i <- lane 7-i within each 8-lane half row
    return x;
}

// Max over the 8 lanes of a slot; every lane receives the same value.
__device__ __forceinline__ float slot_max(float x) {
    x = fmaxf(x, dpp<0xB1>(x));
    x = fmaxf(x, dpp<0x4E>(x));
    return fmaxf(x, dpp<0x141>(x));
}

// Sum / max over the lanes lane ^ m, m = FIRST, 2 FIRST, ..., 32, without the
// LDS crossbar: DPP inside 16-lane rows (FIRST = 1: the slot patterns above,
// then lane ^ 8 = row_ror:8), then the gfx950 row swaps for lane ^ 16 and
// lane ^ 32 (each returns both swapped registers; the pair's sum or max is the
// same whichever way round they come).  Every lane ends with the same bits.
template <int FIRST>
__device__ __forceinline__ float xor_sum(float x) {
    static_assert(FIRST == 1 || FIRST == 8 || FIRST == 16 || FIRST == 32, "lane groups of 1, 8, 16 or 32");
    if constexpr (FIRST == 1) x = slot_sum(x);
    if constexpr (FIRST <= 8) x += dpp<0x128>(x);
    if constexpr (FIRST <= 16) {
        const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    }
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
template <int FIRST>
__device__ __forceinline__ float xor_max(float x) {
    static_assert(FIRST == 1 || FIRST == 8 || FIRST == 16 || FIRST == 32, "lane groups of 1, 8, 16 or 32");
    if constexpr (FIRST == 1) x = slot_max(x);
    if constexpr (FIRST <= 8) x = fmaxf(x, dpp<0x128>(x));
    if constexpr (FIRST <= 16) {
        const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    }
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
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

// A lane's 8 dims of one head: x[0..3] = dims 4c..4c+3, x[4..7] = dims 32+4c..32+4c+3.
__device__ __forceinline__ void load8(float (&x)[8], const float* __restrict__ p) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 32);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

__device__ __forceinline__ void store8(float* __restrict__ p, const float (&x)[8]) {
    *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
    *reinterpret_cast<float4*>(p + 32) = make_float4(x[4], x[5], x[6], x[7]);
}

// 16-bit caches (bf16 / fp16, the same [row][kv][64] layout): a lane's 8 dims
// are two 8-byte loads, widened exactly to fp32; stores round to nearest even.
template <typename T>
__device__ __forceinline__ void load8(float (&x)[8], const T* __restrict__ p) {
    typedef T t4 __attribute__((ext_vector_type(4)));
    const t4 a = *reinterpret_cast<const t4*>(p);
    const t4 b = *reinterpret_cast<const t4*>(p + 32);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        x[t] = (float)a[t];
        x[4 + t] = (float)b[t];
    }
}

template <typename T>
__device__ __forceinline__ void store8(T* __restrict__ p, const float (&x)[8]) {
    typedef T t4 __attribute__((ext_vector_type(4)));
    const t4 a = {(T)x[0], (T)x[1], (T)x[2], (T)x[3]};
    const t4 b = {(T)x[4], (T)x[5], (T)x[6], (T)x[7]};
    *reinterpret_cast<t4*>(p) = a;
    *reinterpret_cast<t4*>(p + 32) = b;
}

// The value a cache of element type T holds for x: what a later read returns,
// so a row attended from registers matches the row attended from memory.
__device__ __forceinline__ void round8(float (&)[8], const float*) {}
template <typename T>
__device__ __forceinline__ void round8(float (&x)[8], const T*) {
#pragma unroll
    for (int t = 0; t < 8; ++t) x[t] = (float)(T)x[t];
}

__device__ __forceinline__ float half_bits_to_float(unsigned h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}

// Q8_0 cache (TMAC_KV_Q8_0).  The 64 dims of one (row, kv head) form a
// 68-byte "head row": int8 q[64], then the fp16 scales d0 (dims 0..31) and d1
// (dims 32..63).  Those are the two 34-byte GGML Q8_0 blocks of the 64 dims
// (value = q * d, as dequant_q8_0 reads them, tmac_gguf.cpp:240-250) with the
// scales moved behind the values, so each lane's 4-dim runs are aligned
// 4-byte words.
struct q8_0_t {};

// Byte geometry of one head row of a cache of element type T.
template <typename T>
struct CacheFmt {
    static constexpr int kHeadBytes = kHeadDim * (int)sizeof(T);
    static constexpr int kDimBytes = (int)sizeof(T);
};
template <>
struct CacheFmt<q8_0_t> {
    static constexpr int kHeadBytes = kQ8HeadBytes;
    static constexpr int kDimBytes = 1;
};

// This lane's 8 dims of a cache head row as loaded (raw words): fp32 8
// floats, 16-bit 4 words, Q8_0 the two 4-byte runs plus the scale word.
// Prefetch buffers hold raw rows and are widened where they are used, so the
// wait for a load sits at its use, not right behind the load.
template <typename T>
struct RawRow {
    unsigned w[sizeof(T) == 2 ? 4 : 3];
};
template <>
struct RawRow<float> {
    float w[8];
};

// A load of a cache word: non-temporal (the `nt` cache policy) when NT.
template <bool NT, typename V>
__device__ __forceinline__ V ld(const char* p) {
    if constexpr (NT)
        return __builtin_nontemporal_load(reinterpret_cast<const V*>(p));
    else
        return *reinterpret_cast<const V*>(p);
}

// p points at the lane's dim 4c of a head row.  The group kernel reads every
// cache row once per launch, so it streams them non-temporally (NT): at
// config 3 that moved the fp32 decode from 185 to 170 us (72% -> 79% of HBM
// peak), the streamed rows no longer displacing useful lines.  The head
// kernel reads each row once per query head, through L2: temporal loads.
template <typename T, bool NT>
__device__ __forceinline__ void load_raw(RawRow<T>& r, const char* p, int c) {
    typedef float f32x4_t __attribute__((ext_vector_type(4)));
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    if constexpr (sizeof(T) == 4) {
        const f32x4_t a = ld<NT, f32x4_t>(p);
        const f32x4_t b = ld<NT, f32x4_t>(p + 32 * sizeof(float));
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            r.w[t] = a[t];
            r.w[4 + t] = b[t];
        }
    } else if constexpr (sizeof(T) == 2) {
        const u32x2 a = ld<NT, u32x2>(p);
        const u32x2 b = ld<NT, u32x2>(p + 32 * sizeof(T));
        r.w[0] = a[0];
        r.w[1] = a[1];
        r.w[2] = b[0];
        r.w[3] = b[1];
    } else {
        r.w[0] = ld<NT, unsigned>(p);               // dims 4c..4c+3
        r.w[1] = ld<NT, unsigned>(p + 32);          // dims 32+4c..32+4c+3
        r.w[2] = ld<NT, unsigned>(p + 64 - 4 * c);  // d0 | d1 << 16
    }
}

// Raw row -> fp32, exactly.
template <typename T>
__device__ __forceinline__ void widen(float (&x)[8], const RawRow<T>& r) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int t = 0; t < 8; ++t) x[t] = r.w[t];
    } else if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            if constexpr (__is_same(T, __bf16)) {
                x[2 * t] = __builtin_bit_cast(float, r.w[t] << 16);
                x[2 * t + 1] = __builtin_bit_cast(float, r.w[t] & 0xFFFF0000u);
            } else {
                x[2 * t] = half_bits_to_float(r.w[t] & 0xFFFFu);
                x[2 * t + 1] = half_bits_to_float(r.w[t] >> 16);
            }
        }
    } else {
        const float d0 = half_bits_to_float(r.w[2] & 0xFFFFu), d1 = half_bits_to_float(r.w[2] >> 16);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            x[t] = (float)(signed char)(r.w[0] >> (8 * t)) * d0;  // |q| <= 127, 11-bit d: exact product
            x[4 + t] = (float)(signed char)(r.w[1] >> (8 * t)) * d1;
        }
    }
}

template <typename T, bool NT>
__device__ __forceinline__ void load_row(float (&x)[8], const char* p, int c) {
    RawRow<T> r;
    load_raw<T, NT>(r, p, c);
    widen<T>(x, r);
}

// fp16 bits of a Q8_0 scale exactly as the reference's converter writes them
// (scripts/extract_tmac.py:53-74): exponent rebased, mantissa truncated to 10
// bits, magnitudes below fp16's normal range flushed to 0, exponents above
// its range turned into infinity.
__device__ __forceinline__ unsigned f16_bits_trunc(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const unsigned e = (u >> 23) & 0xFFu;
    if ((u & 0x7FFFFFFFu) == 0 || e == 0) return 0;
    const unsigned s = (u >> 31) << 15;
    if (e >= 0x8Fu) return s | (31u << 10);
    if (e <= 0x70u) return s;
    return s | ((e - 112u) << 10) | ((u & 0x7FFFFFu) >> 13);
}

// One lane's 4 dims of a 32-dim block quantized as quantize_q8_0_block does
// (scripts/extract_tmac.py:159-173): d = amax / 127 (1 when amax < 1e-10),
// q = x / d rounded half to even, the scale stored as f16_bits_trunc(d).
// amax is the block's max |x|.  Returns the 4 bytes; x becomes what the cache
// then holds, q * fp16(d).
__device__ __forceinline__ unsigned quant4(float* x, float amax, unsigned& dbits) {
    const float d = amax < 1e-10f ? 1.0f : amax / 127.0f;  // IEEE division (hipcc default)
    dbits = f16_bits_trunc(d);
    const float dq = half_bits_to_float(dbits);
    unsigned packed = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int qv = (int)__builtin_rintf(x[t] / d);
        packed |= ((unsigned)qv & 0xFFu) << (8 * t);
        x[t] = (float)qv * dq;
    }
    return packed;
}

// Rounds x (this lane's 8 dims of a new cache head row) to the value a cache
// of type T holds and, if `store`, writes it at p (the lane's dim 4c).
template <typename T>
__device__ __forceinline__ void put_row(float (&x)[8], char* p, int, bool store) {
    round8(x, static_cast<const T*>(nullptr));
    if (store) store8(reinterpret_cast<T*>(p), x);
}
// Q8_0: the 8 lanes of a slot hold the head row's 64 dims and must all call
// (the block maxima are reduced across them); lane 0 writes the scales.
template <>
__device__ __forceinline__ void put_row<q8_0_t>(float (&x)[8], char* p, int c, bool store) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        a0 = fmaxf(a0, fabsf(x[t]));
        a1 = fmaxf(a1, fabsf(x[4 + t]));
    }
    a0 = slot_max(a0);
    a1 = slot_max(a1);
    unsigned d0, d1;
    const unsigned lo = quant4(x, a0, d0);
    const unsigned hi = quant4(x + 4, a1, d1);
    if (store) {
        *reinterpret_cast<unsigned*>(p) = lo;
        *reinterpret_cast<unsigned*>(p + 32) = hi;
        if (c == 0) *reinterpret_cast<unsigned*>(p + 64) = d0 | (d1 << 16);
    }
}

// Paged modes: a sequence's rows live in kPageRows-row pages of a pool, and
// table[j] is the pool page holding its rows kPageRows*j .. kPageRows*j + 15.
// Page indices outside [0, n_pages) are clamped into the pool and reported.
struct PageMap {
    const int32_t* table;  // this sequence's block-table row
    int r0;                // first row of the range being attended (a multiple of kPageRows)
    int n_pages;
};

typedef __attribute__((address_space(4))) const int32_t* const_i32_ptr;

// Pool page of a sequence row (wave-uniform).  The block table is read-only
// for the kernel's lifetime, so it is read through the constant address space
// (a scalar load); a vector load would join the in-order queue of the K/V
// prefetches and wait behind them.
__device__ __forceinline__ unsigned page_of(const PageMap& pm, int row, unsigned& bad) {
    row = __builtin_amdgcn_readfirstlane(row);  // uniform by construction; lets the load be scalar
    const unsigned pg = (unsigned)((const_i32_ptr)pm.table)[row >> kPageShift];
    bad |= pg >= (unsigned)pm.n_pages ? 1u : 0u;
    return min(pg, (unsigned)pm.n_pages - 1u);
}

// RoPE on a lane's 8 dims.  Pairs (d, d+1), d even, never straddle a lane:
// dims 4c..4c+3 are pairs 2c, 2c+1 and dims 32+4c.. are pairs 16+2c, 17+2c.
__device__ __forceinline__ void rope8(float (&x)[8], const float2* __restrict__ cs_row, int c) {
    const float4 t0 = *reinterpret_cast<const float4*>(cs_row + 2 * c);
    const float4 t1 = *reinterpret_cast<const float4*>(cs_row + 16 + 2 * c);
    rotate_pair(x[0], x[1], t0.x, t0.y);
    rotate_pair(x[2], x[3], t0.z, t0.w);
    rotate_pair(x[4], x[5], t1.x, t1.y);
    rotate_pair(x[6], x[7], t1.z, t1.w);
}

// RoPE row of a layer step through the position counter's row cache
// (DecodeArgs::pos_slots, filled by tmac_pos_update): both slots are read
// together with the position, and the row is read from the table only when
// neither slot is tagged with (position, table), so the q / k rotation need
// not wait for the position.
struct RopePrefetch {
    float4 a0, b0, a1, b1;          // lane c's pairs 2c, 2c+1 and 16+2c, 16+2c+1 of slots 0 and 1
    int tag0, lo0, hi0, tag1, lo1, hi1;
};
__device__ __forceinline__ RopePrefetch rope_prefetch(const DecodeArgs& a, int c) {
    RopePrefetch p;
    p.a0 = p.b0 = p.a1 = p.b1 = make_float4(0.f, 0.f, 0.f, 0.f);
    p.tag0 = p.tag1 = -1;
    p.lo0 = p.hi0 = p.lo1 = p.hi1 = 0;
    if (a.pos_slots) {
        const float2* s = a.pos_slots;
        p.a0 = *reinterpret_cast<const float4*>(s + 2 * c);
        p.b0 = *reinterpret_cast<const float4*>(s + 16 + 2 * c);
        p.a1 = *reinterpret_cast<const float4*>(s + 32 + 2 * c);
        p.b1 = *reinterpret_cast<const float4*>(s + 48 + 2 * c);
        const int* tag = reinterpret_cast<const int*>(s + 64);
        p.tag0 = tag[0]; p.lo0 = tag[1]; p.hi0 = tag[2];
        p.tag1 = tag[4]; p.lo1 = tag[5]; p.hi1 = tag[6];
    }
    return p;
}
__device__ __forceinline__ void rope_pairs(const DecodeArgs& a, const RopePrefetch& p, int pos, int c, float4& t0,
                                           float4& t1) {
    const uint64_t tab = reinterpret_cast<uint64_t>(a.rope_cs);
    const int lo = (int)(uint32_t)tab, hi = (int)(uint32_t)(tab >> 32);
    const bool h0 = p.tag0 == pos && p.lo0 == lo && p.hi0 == hi;
    const bool h1 = p.tag1 == pos && p.lo1 == lo && p.hi1 == hi;
    if (h0 || h1) {
        t0.x = h0 ? p.a0.x : p.a1.x; t0.y = h0 ? p.a0.y : p.a1.y;
        t0.z = h0 ? p.a0.z : p.a1.z; t0.w = h0 ? p.a0.w : p.a1.w;
        t1.x = h0 ? p.b0.x : p.b1.x; t1.y = h0 ? p.b0.y : p.b1.y;
        t1.z = h0 ? p.b0.z : p.b1.z; t1.w = h0 ? p.b0.w : p.b1.w;
    } else {
        const float2* row = a.rope_cs + (size_t)pos * (kHeadDim / 2);
        t0 = *reinterpret_cast<const float4*>(row + 2 * c);
        t1 = *reinterpret_cast<const float4*>(row + 16 + 2 * c);
        // (waited for here, so that after the branch the compiler waits for
        // the slot loads alone, not for every load issued since them)
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
}
// rope8 with the lane's pairs already loaded
__device__ __forceinline__ void rope8p(float (&x)[8], const float4& t0, const float4& t1) {
    rotate_pair(x[0], x[1], t0.x, t0.y);
    rotate_pair(x[2], x[3], t0.z, t0.w);
    rotate_pair(x[4], x[5], t1.x, t1.y);
    rotate_pair(x[6], x[7], t1.z, t1.w);
}
template <int G>
struct State {
    float m[G];                // running max (log2 domain), identical across a kv group's lanes
    float l[G];                // running sum of weights
    float acc[G][kDimsPerLane];// running sum of weight * v over this lane's dims
};

template <int G>
__device__ __forceinline__ void state_init(State<G>& st) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
        st.m[g] = kNegInf;
        st.l[g] = 0.f;
#pragma unroll
        for (int t = 0; t < kDimsPerLane; ++t) st.acc[g][t] = 0.f;
    }
}

// One step: this lane's slot sees one cache row (kf/vf = its 8 dims of the
// row's kv head) or nothing (valid == false; only when MASKED).
template <int G, int KV, bool MASKED>
__device__ __forceinline__ void attend(const float (&q)[G][kDimsPerLane], State<G>& st,
                                       const float (&kf)[kDimsPerLane], const float (&vf)[kDimsPerLane],
                                       bool valid) {
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float a = q[g][0] * kf[0];
#pragma unroll
        for (int t = 1; t < kDimsPerLane; ++t) a = fmaf(q[g][t], kf[t], a);
        s[g] = slot_sum(a);
        if (MASKED) s[g] = valid ? s[g] : kNegInf;
    }
    float over = s[0] - st.m[0];
#pragma unroll
    for (int g = 1; g < G; ++g) over = fmaxf(over, s[g] - st.m[g]);
    if (__any(over > kTau)) {
        // Raise the wave's shared max to this step's max (rare after the first step).
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mx = xor_max<kLanesPerSlot * KV>(s[g]);
            const float mn = fmaxf(st.m[g], mx);
            const float alpha = (st.m[g] == kNegInf) ? 0.f : fast_exp2(st.m[g] - mn);
            st.l[g] *= alpha;
#pragma unroll
            for (int t = 0; t < kDimsPerLane; ++t) st.acc[g][t] *= alpha;
            st.m[g] = mn;
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float e = fast_exp2(s[g] - st.m[g]);  // 0 for masked slots (s = -inf)
        st.l[g] += e;
#pragma unroll
        for (int t = 0; t < kDimsPerLane; ++t) st.acc[g][t] = fmaf(e, vf[t], st.acc[g][t]);
    }
}

// Attends this wave's share of `n_rows` cache rows starting at kb/vb.  A step
// covers PPS = 8/KVS rows x KVS kv heads (ROWB bytes between rows).  Steps are
// dealt round-robin to the NW waves of the workgroup (the workgroup streams its
// range front to back); DEPTH steps of K/V are kept in flight per wave.  Full
// steps run in the main loop; the one partial step at the end of the range (if
// any) is loaded and masked after it, so the loop body holds a single copy of
// the softmax state.  PAGED: kb/vb are the pool bases and pm maps rows to
// pages (PPS divides kPageRows and pm.r0 is page-aligned, so a step never
// straddles a page).
template <typename T, int G, int KVS, int ROWB, int NW, int DEPTH, bool PAGED>
__device__ __forceinline__ void attend_rows(const char* __restrict__ kb, const char* __restrict__ vb,
                                            int n_rows, int wave, int lane_off, int lane_row,
                                            int lane_col, int c, const float (&q)[G][kDimsPerLane],
                                            State<G>& st, int rot, bool blocked, const PageMap& pm,
                                            unsigned& bad) {
    constexpr int PPS = kSlots / KVS;   // rows per step
    constexpr int STEP = PPS * ROWB;    // bytes between consecutive steps
    static_assert(kPageRows % PPS == 0, "a step must not straddle a page");
    const int full = n_rows / PPS;      // steps whose rows are all in range
    // Interleaved: wave w takes steps w, w + NW, ...  Blocked: wave w takes a
    // contiguous run of steps (NW independent streams per workgroup).
    int first, nk, stride;
    if (blocked) {
        const int per = (full + NW - 1) / NW;
        first = wave * per;
        nk = max(min(full - first, per), 0);
        stride = 1;
    } else {
        first = wave;
        nk = (full - wave + NW - 1) / NW;
        stride = NW;
    }

    if (nk > 0) {
        // The wave visits its steps starting `rot` steps in and wrapping, so that
        // concurrently running workgroups stream from staggered offsets of their
        // ranges (spreads the HBM channels; the merge is order-independent).
        rot %= nk;
        RawRow<T> kbuf[DEPTH], vbuf[DEPTH];
        const char* kp = kb + (PAGED ? 0 : (size_t)first * STEP) + lane_off;
        const char* vp = vb + (PAGED ? 0 : (size_t)first * STEP) + lane_off;
        auto at = [&](int k) -> size_t {
            int kk = k + rot;
            kk -= (kk >= nk) ? nk : 0;
            if (!PAGED) return (size_t)kk * stride * STEP;
            const int row = pm.r0 + (first + kk * stride) * PPS;
            return ((size_t)page_of(pm, row, bad) * kPageRows + (row & (kPageRows - 1))) * ROWB;
        };
        // Prefetches are unconditional (indices past the wave's last step are
        // clamped to it, an L2 hit), so every buffer keeps one register
        // assignment across iterations; a conditional load would make the
        // compiler rotate buffers with copies, which must first wait for all
        // loads in flight.
        // The prologue issues step 0 first, then step 1, ... (the scheduling
        // barrier keeps that order).  The wait at the loop head covers both
        // the loop entry and the back edge, so with another prologue order
        // the entry path forces a wait for (nearly) every load in flight on
        // every iteration (2% slower at config 3 with an fp32 cache, 4% with
        // a bf16 cache).
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            load_raw<T, true>(kbuf[d], kp + at(min(d, nk - 1)), c);
            load_raw<T, true>(vbuf[d], vp + at(min(d, nk - 1)), c);
            __builtin_amdgcn_sched_barrier(0);
        }
        for (int k0 = 0; k0 < nk; k0 += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                if (k0 + d < nk) {
                    float kf[kDimsPerLane], vf[kDimsPerLane];
                    widen<T>(kf, kbuf[d]);
                    widen<T>(vf, vbuf[d]);
                    attend<G, KVS, false>(q, st, kf, vf, true);
                }
                const int kn = min(k0 + d + DEPTH, nk - 1);
                load_raw<T, true>(kbuf[d], kp + at(kn), c);
                load_raw<T, true>(vbuf[d], vp + at(kn), c);
            }
        }
    }
    if (full * PPS < n_rows && (full % NW) == wave) {
        const int row = full * PPS + lane_row;
        const int r = min(row, n_rows - 1);  // in the same step (and page) as row full * PPS
        size_t off;
        if (PAGED)
            off = ((size_t)page_of(pm, pm.r0 + full * PPS, bad) * kPageRows + ((pm.r0 + r) & (kPageRows - 1))) *
                      ROWB + lane_col;
        else
            off = (size_t)r * ROWB + lane_col;
        float kf[kDimsPerLane], vf[kDimsPerLane];
        load_row<T, true>(kf, kb + off, c);
        load_row<T, true>(vf, vb + off, c);
        attend<G, KVS, true>(q, st, kf, vf, row < n_rows);
    }
}

// Merges NW partial states (acc over 64 dims, base-2 max m, sum l) held in
// LDS, one thread per (head, dim) with the block's NT threads striding over
// them, and writes the output (single split) or this split's (acc, m, l)
// partial.  The caller synchronizes first.
template <int NH, int NW, int NT>
__device__ __forceinline__ void merge_waves(const float (*s_acc)[NH][kHeadDim], const float (*s_m)[NH],
                                            const float (*s_l)[NH], bool direct, float* __restrict__ out_heads,
                                            float* __restrict__ ws_split) {
    for (int idx = threadIdx.x; idx < NH * kHeadDim; idx += NT) {
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
            out_heads[idx] = A / L;
        } else {
            float* p = ws_split + (size_t)h * kPartialStride;
            p[d] = A;
            if (d == 0) {
                p[kHeadDim] = M;
                p[kHeadDim + 1] = L;
            }
        }
    }
}

// Merges one workgroup's NW wave states (KVS*G heads) and writes either the
// final output (single split) or this split's (acc, m, l) partial.
template <int G, int KVS, int NW>
__device__ __forceinline__ void finish(State<G>& st, int lane, int wave, bool direct,
                                       float* __restrict__ out_heads, float* __restrict__ ws_split) {
    constexpr int NH = KVS * G;
    // 1. Sum the slots of each kv group inside the wave (they share the max).
#pragma unroll
    for (int g = 0; g < G; ++g) {
        st.l[g] = xor_sum<kLanesPerSlot * KVS>(st.l[g]);
#pragma unroll
        for (int t = 0; t < kDimsPerLane; ++t) st.acc[g][t] = xor_sum<kLanesPerSlot * KVS>(st.acc[g][t]);
    }
    // 2. Waves -> LDS.
    __shared__ float s_acc[NW][NH][kHeadDim];
    __shared__ float s_m[NW][NH];
    __shared__ float s_l[NW][NH];
    const int slot = lane / kLanesPerSlot, c = lane % kLanesPerSlot;
    if (slot < KVS) {  // row 0 of the step holds the wave total for kv slot `slot`
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int h = slot * G + g;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s_acc[wave][h][4 * c + j] = st.acc[g][j];
                s_acc[wave][h][32 + 4 * c + j] = st.acc[g][4 + j];
            }
            if (c == 0) {
                s_m[wave][h] = st.m[g];
                s_l[wave][h] = st.l[g];
            }
        }
    }
    __syncthreads();
    merge_waves<NH, NW, NW * 64>(s_acc, s_m, s_l, direct, out_heads, ws_split);
}

// Rows attended by sequence `seq` (n_pos) and its first cache row (base;
// 0 in the layer and paged modes), per mode.  Returns false for an
// out-of-range position.
template <int MODE>
__device__ __forceinline__ bool seq_geometry(const DecodeArgs& a, int seq, int& n_pos, int& pos,
                                             size_t& base) {
    pos = 0;
    base = 0;
    if (MODE == kUniform) {
        n_pos = a.n_pos;
        base = (size_t)seq * (size_t)a.seq_stride;
    } else if (MODE == kRagged) {
        n_pos = a.lengths[seq];
        base = (size_t)a.offsets[seq];
    } else if (MODE == kPaged) {
        n_pos = a.lengths[seq];
    } else {
        pos = MODE == kPagedLayer ? a.positions[seq] : (a.pos_dev ? *a.pos_dev : a.pos_host);
        if (pos < 0 || pos >= a.capacity || pos >= a.rope_rows) return false;
        n_pos = pos + 1;
    }
    return true;
}

// Flat unit grid (ragged and paged modes): unit index -> (sequence, split).
// Sequence s with L_s = lengths[s] + add rows owns
// clamp(ceil(L_s / split_len), 1, n_splits) consecutive units (a length above
// the launch's max_len still gets its units, whose first one reports it), so
// the unit count never exceeds the n_seq * n_splits grid; the units that carry
// rows fill the front of the grid (round-robin dispatch then spreads them
// evenly over the XCDs) and surplus workgroups at the end exit.  Every wave
// computes the same answer: lane l takes kScanPer consecutive sequences of a
// round of 64 * kScanPer (their loads, and those of their `offsets` entries
// when given, all in flight at once), and a 64-lane inclusive scan of the lane
// sums finds the lane, then the sequence, holding the unit.  The sequence's
// array value (raw) and offset come back with it, so the caller needs no
// second round trip to memory before its K/V addresses are known.
constexpr int kScanPer = 8;

// Inclusive prefix sum over the 64 lanes: DPP row shifts inside each 16-lane
// row, then the row totals read from lanes 15, 31 and 47.
__device__ __forceinline__ int wave_incl_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1 (lanes shifted in add 0)
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
    const int r0 = __builtin_amdgcn_readlane(x, 15), r1 = __builtin_amdgcn_readlane(x, 31);
    const int r2 = __builtin_amdgcn_readlane(x, 47);
    const int row = (threadIdx.x & 63) >> 4;
    return x + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}

__device__ __forceinline__ bool ragged_unit(const int32_t* __restrict__ lengths,
                                            const int64_t* __restrict__ offsets, int add, int n_seq, int split_len,
                                            int n_splits, int unit, int& seq, int& split, int& raw, int64_t& off) {
    const int lane = threadIdx.x & 63;
    int base = 0;
    for (int c0 = 0; c0 < n_seq; c0 += 64 * kScanPer) {
        const int s0 = c0 + lane * kScanPer;
        int v[kScanPer];
        int64_t o[kScanPer];
#pragma unroll
        for (int j = 0; j < kScanPer; ++j) {
            const bool in = s0 + j < n_seq;
            v[j] = in ? lengths[s0 + j] : 0;
            o[j] = (in && offsets) ? offsets[s0 + j] : 0;
        }
        int u[kScanPer];
        int sum = 0;
#pragma unroll
        for (int j = 0; j < kScanPer; ++j) {
            // rows L = v + add (add is 0 or 1, so L fits 32 unsigned bits); ceil(L / split_len), 1 for L <= 0
            const int64_t len = (int64_t)v[j] + add;
            unsigned uu = 1;
            if (len > 0) uu = ((unsigned)len - 1u) / (unsigned)split_len + 1u;
            u[j] = s0 + j < n_seq ? (int)min(uu, (unsigned)n_splits) : 0;
            sum += u[j];
        }
        const int incl = wave_incl_scan(sum);
        const int total = __builtin_amdgcn_readlane(incl, 63);
        if (unit < base + total) {
            const unsigned long long hit = __ballot(unit < base + incl);
            const int first = __builtin_amdgcn_readfirstlane(__ffsll((long long)hit) - 1);
            // Every lane resolves the unit inside its own sequences as if it
            // were the hit lane; the hit lane's answer is read out.
            int e = base + incl - sum, jj = 0, sp = 0, vv = v[0];
            int64_t oo = o[0];
#pragma unroll
            for (int j = 0; j < kScanPer; ++j) {
                if (unit >= e && unit < e + u[j]) {
                    jj = j;
                    sp = unit - e;
                    vv = v[j];
                    oo = o[j];
                }
                e += u[j];
            }
            seq = __builtin_amdgcn_readlane(s0 + jj, first);
            split = __builtin_amdgcn_readlane(sp, first);
            raw = __builtin_amdgcn_readlane(vv, first);
            const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(uint32_t)oo, first);
            const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)oo >> 32), first);
            off = (int64_t)(((uint64_t)hi << 32) | lo);
            return seq >= 0 && seq < n_seq && split >= 0 && split < n_splits;
        }
        base += total;
    }
    return false;
}

// Geometry of a unit-grid sequence from the values ragged_unit read:
// raw = lengths[seq] (ragged, paged) or positions[seq] (paged layer).
template <int MODE>
__device__ __forceinline__ bool unit_geometry(const DecodeArgs& a, int raw, int64_t off, int& n_pos, int& pos,
                                              size_t& base) {
    pos = 0;
    base = 0;
    if (MODE == kRagged) {
        n_pos = raw;
        base = (size_t)off;
    } else if (MODE == kPaged) {
        n_pos = raw;
    } else {
        pos = raw;
        if (pos < 0 || pos >= a.capacity || pos >= a.rope_rows) return false;
        n_pos = pos + 1;
    }
    return true;
}

// Decode for one (split, sequence) workgroup.
//   PER_HEAD = false ("group" kernel): grid (split, seq); every lane carries
//     the G query heads of its kv head and a step covers all KV kv heads of
//     PPS = 8/KV rows, so each K/V byte is read from memory once.
//   PER_HEAD = true ("head" kernel, short contexts): grid (q head, seq), one
//     split; the workgroup attends all rows for one query head, reading only
//     its kv head's 256-byte half rows, so no cross-workgroup merge is needed.
// Ragged and paged modes launch a flat unit grid instead of (split, seq).
// The paged layer mode is the layer step of a batch: sequence s's new token
// sits at positions[s], and its q/k_new/v_new rows are the s-th of each input.
template <typename T, int G, int KV, int NW, int DEPTH, int MODE, bool PER_HEAD>
__device__ __forceinline__ void decode_body(const DecodeArgs& a) {
    constexpr int HB = CacheFmt<T>::kHeadBytes;
    constexpr int ROWB = KV * HB;            // cache bytes per row
    constexpr int ROWF = KV * kHeadDim;      // floats per k_new / v_new row
    constexpr int NH = KV * G;
    constexpr int KVS = PER_HEAD ? 1 : KV;  // kv heads per step
    constexpr int GW = PER_HEAD ? 1 : G;    // query heads per lane
    constexpr bool PAGED = is_paged(MODE);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int split = PER_HEAD ? 0 : blockIdx.x;
    const int head = PER_HEAD ? blockIdx.x : 0;
    int seq = blockIdx.y;
    int n_pos, pos;
    size_t base;
    bool geo_ok;
    if ((MODE == kRagged || PAGED) && !PER_HEAD) {  // grid = flat list of (sequence, split) units
        const bool by_pos = MODE == kPagedLayer;
        int raw;
        int64_t off;
        if (!ragged_unit(by_pos ? a.positions : a.lengths, MODE == kRagged ? a.offsets : nullptr, by_pos ? 1 : 0,
                         a.n_seq, a.split_len, a.n_splits, blockIdx.x, seq, split, raw, off))
            return;
        geo_ok = unit_geometry<MODE>(a, raw, off, n_pos, pos, base);
    } else {
        geo_ok = seq_geometry<MODE>(a, seq, n_pos, pos, base);
    }
    if (!geo_ok) {
        if (split == 0 && threadIdx.x == 0) atomicOr(a.err, 1);
        return;
    }
    // Per-sequence values are uniform; read from memory (ragged, paged modes)
    // they would otherwise stay in vector registers, and so would all the
    // address arithmetic derived from them.
    n_pos = __builtin_amdgcn_readfirstlane(n_pos);
    pos = __builtin_amdgcn_readfirstlane(pos);
    float* out_seq = a.out + (size_t)seq * NH * kHeadDim;
    float* out_heads = out_seq + (PER_HEAD ? head * kHeadDim : 0);
    if (n_pos <= 0) {  // ragged sequence with no rows: defined as a zero output
        if (split == 0)
            for (int i = threadIdx.x; i < KVS * GW * kHeadDim; i += NW * 64) out_heads[i] = 0.f;
        return;
    }
    const int n_act = (n_pos + a.split_len - 1) / a.split_len;
    if (n_act > a.n_splits) {  // length above the max_len the grid was sized for
        if (split == 0) {
            for (int i = threadIdx.x; i < KVS * GW * kHeadDim; i += NW * 64) out_heads[i] = __builtin_nanf("");
            if (threadIdx.x == 0) atomicOr(a.err, 2);
        }
        return;
    }
    if (split >= n_act) return;
    const int mem_rows = is_layer(MODE) ? pos : n_pos;  // layer modes: row `pos` comes from registers
    const int r0 = split * a.split_len;
    const int r1 = min(r0 + a.split_len, mem_rows);

    const int slot = lane / kLanesPerSlot, c = lane % kLanesPerSlot;
    const int lane_row = slot / KVS;
    const int kvh = PER_HEAD ? head / G : slot % KVS;  // kv head this lane reads
    const int lane_colf = kvh * kHeadDim + 4 * c;                     // in fp32 inputs
    const int lane_col = kvh * HB + 4 * c * CacheFmt<T>::kDimBytes;   // in a cache row (bytes)
    const int lane_off = lane_row * ROWB + lane_col;

    // Query of this lane's GW heads (its 8 dims), pre-scaled for base-2 softmax.
    float q[GW][kDimsPerLane];
    const float2* cs_row = nullptr;
    if (is_layer(MODE)) cs_row = a.rope_cs + (size_t)pos * (kHeadDim / 2);
#pragma unroll
    for (int g = 0; g < GW; ++g) {
        const int qh = PER_HEAD ? head : kvh * G + g;
        load8(q[g], a.q + ((size_t)seq * NH + qh) * kHeadDim + 4 * c);
        if (is_layer(MODE)) rope8(q[g], cs_row, c);
#pragma unroll
        for (int t = 0; t < kDimsPerLane; ++t) q[g][t] *= a.qscale;
    }

    State<GW> st;
    state_init(st);
    const char* kc = reinterpret_cast<const char*>(a.k) + (PAGED ? 0 : (base + r0) * ROWB);
    const char* vc = reinterpret_cast<const char*>(a.v) + (PAGED ? 0 : (base + r0) * ROWB);
    const PageMap pm{PAGED ? a.block_table + (size_t)seq * a.max_pages : nullptr, r0, a.n_pages};
    unsigned bad = 0;
    attend_rows<T, GW, KVS, ROWB, NW, DEPTH, PAGED>(kc, vc, max(r1 - r0, 0), wave, lane_off, lane_row, lane_col, c,
                                                   q, st, (blockIdx.y * gridDim.x + blockIdx.x) * a.rot_mul,
                                                   a.blocked != 0, pm, bad);

    if (is_layer(MODE) && split == n_act - 1 && wave == 0) {
        // The new token (row `pos`): RoPE its k, write k/v to the cache row
        // (tmac_gguf.cpp:1090-1091, once per kv head) and attend it from registers.
        const bool mine = (lane_row == 0);
        float kf[kDimsPerLane], vf[kDimsPerLane];
        if (mine) {
            const size_t in = (MODE == kPagedLayer ? (size_t)seq * ROWF : 0) + lane_colf;
            load8(kf, a.k_new + in);
            load8(vf, a.v_new + in);
            rope8(kf, cs_row, c);
            size_t row = (size_t)pos;
            if (PAGED) row = (size_t)page_of(pm, pos, bad) * kPageRows + (pos & (kPageRows - 1));
            const bool store = !PER_HEAD || head % G == 0;
            put_row<T>(kf, reinterpret_cast<char*>(a.k_out) + row * ROWB + lane_col, c, store);
            put_row<T>(vf, reinterpret_cast<char*>(a.v_out) + row * ROWB + lane_col, c, store);
        } else {
#pragma unroll
            for (int t = 0; t < kDimsPerLane; ++t) kf[t] = vf[t] = 0.f;
        }
        attend<GW, KVS, true>(q, st, kf, vf, mine);
    }
    if (PAGED && bad && lane == 0) atomicOr(a.err, 4);

    const bool direct = (n_act == 1);
    float* ws_split = direct ? nullptr : a.ws + ((size_t)seq * a.n_splits + split) * NH * kPartialStride;
    finish<GW, KVS, NW>(st, lane, wave, direct, out_heads, ws_split);
}

// Rows a ragged sequence of length `len` occupies in the stream-K row space:
// rounded up to kPageRows, and none for an empty sequence or one longer than
// the launch's max_len (its output is written by the combine).
__device__ __forceinline__ int64_t sk_rows(int len, int max_len) {
    return (len > 0 && len <= max_len) ? (((int64_t)len + kPageRows - 1) & ~(int64_t)(kPageRows - 1)) : 0;
}

// Rows attended by sequence s: its length, or in the layer step position + 1
// (0 for a position outside the cache or the RoPE table, which the combine
// reports).
template <bool LAYER>
__device__ __forceinline__ int sk_len(const DecodeArgs& a, int s) {
    if (!LAYER) return a.lengths[s];
    const int pos = a.positions[s];
    return (pos < 0 || pos >= a.capacity || pos >= a.rope_rows) ? 0 : pos + 1;
}

// Stream-K ragged decode.  The batch's sequences, each padded to a multiple of
// kPageRows rows, are laid end to end in one row space of R rows, cut into
// gridDim.x equal ranges of S = max(ceil(R / gridDim.x) rounded up to
// kPageRows, kSkMinRows) rows; workgroup u attends the part of every sequence
// that falls in [u*S, (u+1)*S).  Every workgroup thus streams the same number
// of bytes whatever the length mix, and equal lengths that divide evenly give
// one sequence per workgroup.
// The segment (sequence s, workgroup u) writes its partial to slot u + s of
// the workspace.  Slots are unique: when u - 1 reaches sequence s + 1, u
// starts after s.  Sequence s owns the consecutive slots uf + s .. ul + s
// (uf, ul: the workgroups holding its first and last rows), and workgroup uf
// records (uf + s, ul - uf + 1) in seg_meta[s] for the combine.  A sequence
// inside one workgroup's range is written to the output directly.
// Paged caches: ranges and segments start at multiples of kPageRows, so a
// step or tile never straddles a page.
constexpr int kSkMinRows = 64;

// This workgroup's range [lo, hi) of the row space, S, the last workgroup
// with rows, and the sequence holding row lo with its first row (s0, P0).
// False when the row space ends before the range.  NT threads, all of which
// must call it.
template <int NT, bool LAYER>
__device__ __forceinline__ bool sk_locate(const DecodeArgs& a, int64_t& S, int64_t& lo, int64_t& hi, int& last_u,
                                          int& s0, int64_t& P0) {
    constexpr int NW = NT / 64;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    __shared__ int64_t s_wsum[NW];
    __shared__ int64_t s_hit[2];  // (sequence, its first row)

    // 1. R: every thread sums the padded lengths of sequences t, t + NT, ...;
    //    the first kKeep rounds' values stay in registers for the search below
    //    (their loads are all issued before any is used).
    constexpr int kKeep = 4;
    int64_t kept[kKeep];
#pragma unroll
    for (int r = 0; r < kKeep; ++r) {
        const int sq = r * NT + (int)threadIdx.x;
        kept[r] = sq < a.n_seq ? sk_rows(sk_len<LAYER>(a, sq), a.sk_max_len) : 0;
    }
    int64_t mine = 0;
#pragma unroll
    for (int r = 0; r < kKeep; ++r) mine += kept[r];
#pragma unroll 8
    for (int sq = (int)threadIdx.x + kKeep * NT; sq < a.n_seq; sq += NT)
        mine += sk_rows(sk_len<LAYER>(a, sq), a.sk_max_len);
#pragma unroll
    for (int mask = 1; mask < 64; mask <<= 1) mine += __shfl_xor(mine, mask);
    if (lane == 0) s_wsum[wave] = mine;
    if (threadIdx.x == 0) s_hit[0] = -1;
    __syncthreads();
    int64_t R = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) R += s_wsum[w];
    S = (R + gridDim.x - 1) / gridDim.x;
    S = max((S + kPageRows - 1) & ~(int64_t)(kPageRows - 1), (int64_t)kSkMinRows);
    lo = (int64_t)blockIdx.x * S;
    hi = lo + S;
    last_u = (int)min((R - 1) / S, (int64_t)gridDim.x - 1);
    if (lo >= R) return false;  // uniform: every thread has the same R
    __syncthreads();            // s_wsum is reused below

    // 2. The sequence holding row lo, and its first row: a workgroup-wide
    //    inclusive scan of the padded lengths, NT sequences per round, until a
    //    round contains lo.
    int64_t base = 0;
    for (int c0 = 0, r = 0; c0 < a.n_seq; c0 += NT, ++r) {
        const int sq = c0 + (int)threadIdx.x;
        int64_t rows = 0;
        if (r < kKeep) {
#pragma unroll
            for (int j = 0; j < kKeep; ++j) rows = j == r ? kept[j] : rows;
        } else {
            rows = sq < a.n_seq ? sk_rows(sk_len<LAYER>(a, sq), a.sk_max_len) : 0;
        }
        int64_t incl = rows;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int64_t t = __shfl_up(incl, off);
            if (lane >= off) incl += t;
        }
        if (lane == 63) s_wsum[wave] = incl;
        __syncthreads();
        int64_t before = base, total = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const int64_t x = s_wsum[w];
            before += w < wave ? x : 0;
            total += x;
        }
        const int64_t first = before + incl - rows;
        if (rows > 0 && first <= lo && lo < first + rows) {
            s_hit[0] = sq;
            s_hit[1] = first;
        }
        __syncthreads();  // also orders this round's s_wsum reads before the next round's writes
        if (s_hit[0] >= 0) break;
        base += total;
    }
    s0 = (int)s_hit[0];
    P0 = s_hit[1];
    return true;
}

// Advances (s, P) to the first sequence from s on with rows in [lo, hi)
// (P: its first row in the row space, len: its length); false when there is
// none.  The values are uniform, so they are kept in scalar registers.
template <bool LAYER>
__device__ __forceinline__ bool sk_seek(const DecodeArgs& a, int64_t lo, int64_t hi, int& s, int64_t& P, int& len) {
    for (; s < a.n_seq && P < hi; ++s) {
        s = __builtin_amdgcn_readfirstlane(s);
        len = __builtin_amdgcn_readfirstlane(sk_len<LAYER>(a, s));
        const int64_t rows = sk_rows(len, a.sk_max_len);
        if (rows > 0 && lo - P < (int64_t)len) return true;  // lo - P < len: a row of s lies in [lo, hi)
        P += rows;
    }
    return false;
}

// The combine's record for sequence s (first workspace slot, slots used),
// written by the workgroup holding its first row; returns true when the
// sequence lies inside this workgroup's range (its output is written
// directly).  Segment slot of workgroup u: u + s.
__device__ __forceinline__ bool sk_record(const DecodeArgs& a, int s, int64_t P, int len, int64_t S, int last_u) {
    const int uf = (int)min(P / S, (int64_t)last_u);
    const int ul = (int)min((P + len - 1) / S, (int64_t)last_u);
    if ((int)blockIdx.x == uf && threadIdx.x == 0) {
        a.seg_meta[2 * s] = uf + s;
        a.seg_meta[2 * s + 1] = ul - uf + 1;
    }
    return uf == ul;
}

// Stream-K decode, VALU group kernel (fp32 caches).  The next segment's query
// is loaded before this one's merge, so its latency overlaps the merge.
// LAYER (paged layer step of a batch): sequence s attends rows 0..positions[s];
// the segment holding row positions[s] takes the new token as the unit-grid
// layer kernel does (RoPE of k, the cache row written, attended from registers).
template <typename T, int G, int KV, int NW, int DEPTH, bool PAGED, bool LAYER>
__device__ __forceinline__ void decode_sk_body(const DecodeArgs& a) {
    constexpr int HB = CacheFmt<T>::kHeadBytes;
    constexpr int ROWB = KV * HB;
    constexpr int ROWF = KV * kHeadDim;  // floats per k_new / v_new row
    constexpr int NH = KV * G;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int u = blockIdx.x;
    int64_t S, lo, hi, P;
    int last_u, s, len = 0;
    if (!sk_locate<NW * 64, LAYER>(a, S, lo, hi, last_u, s, P)) return;
    if (!sk_seek<LAYER>(a, lo, hi, s, P, len)) return;

    const int slot = lane / kLanesPerSlot, c = lane % kLanesPerSlot;
    const int lane_row = slot / KV;
    const int kvh = slot % KV;
    const int lane_col = kvh * HB + 4 * c * CacheFmt<T>::kDimBytes;
    const int lane_off = lane_row * ROWB + lane_col;
    auto load_q = [&](float (&q)[G][kDimsPerLane], int sq) {
#pragma unroll
        for (int g = 0; g < G; ++g) load8(q[g], a.q + ((size_t)sq * NH + kvh * G + g) * kHeadDim + 4 * c);
    };
    float q[G][kDimsPerLane];
    load_q(q, s);
    while (true) {
        const int pos = len - 1;  // layer step: the new token's row
        const float2* cs_row = LAYER ? a.rope_cs + (size_t)pos * (kHeadDim / 2) : nullptr;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (LAYER) rope8(q[g], cs_row, c);
#pragma unroll
            for (int t = 0; t < kDimsPerLane; ++t) q[g][t] *= a.qscale;
        }
        const int64_t r0 = max(lo - P, (int64_t)0), r1 = min(hi - P, (int64_t)len);
        const int64_t mem_end = LAYER ? min(r1, (int64_t)pos) : r1;  // layer step: row pos comes from registers
        State<G> st;
        state_init(st);
        const size_t row0 = PAGED ? 0 : (size_t)a.offsets[s] + (size_t)r0;
        const char* kc = reinterpret_cast<const char*>(a.k) + row0 * ROWB;
        const char* vc = reinterpret_cast<const char*>(a.v) + row0 * ROWB;
        const PageMap pm{PAGED ? a.block_table + (size_t)s * a.max_pages : nullptr, (int)r0, a.n_pages};
        unsigned bad = 0;
        attend_rows<T, G, KV, ROWB, NW, DEPTH, PAGED>(kc, vc, (int)max(mem_end - r0, (int64_t)0), wave, lane_off,
                                                     lane_row, lane_col, c, q, st, u * a.rot_mul, a.blocked != 0, pm,
                                                     bad);
        if (LAYER && r1 == len && wave == 0) {
            // The new token: RoPE its k, write k/v to the cache row pos
            // (tmac_gguf.cpp:1090-1091) and attend it from registers.
            const bool mine = (lane_row == 0);
            float kf[kDimsPerLane], vf[kDimsPerLane];
            if (mine) {
                const size_t in = (size_t)s * ROWF + kvh * kHeadDim + 4 * c;
                load8(kf, a.k_new + in);
                load8(vf, a.v_new + in);
                rope8(kf, cs_row, c);
                size_t row = (size_t)pos;
                if (PAGED) row = (size_t)page_of(pm, pos, bad) * kPageRows + (pos & (kPageRows - 1));
                put_row<T>(kf, reinterpret_cast<char*>(a.k_out) + row * ROWB + lane_col, c, true);
                put_row<T>(vf, reinterpret_cast<char*>(a.v_out) + row * ROWB + lane_col, c, true);
            } else {
#pragma unroll
                for (int t = 0; t < kDimsPerLane; ++t) kf[t] = vf[t] = 0.f;
            }
            attend<G, KV, true>(q, st, kf, vf, mine);
        }
        if (PAGED && bad && lane == 0) atomicOr(a.err, 4);
        const bool direct = sk_record(a, s, P, len, S, last_u);
        int s2 = s + 1, len2 = 0;
        int64_t P2 = P + sk_rows(len, a.sk_max_len);
        const bool more = sk_seek<LAYER>(a, lo, hi, s2, P2, len2);
        if (more) load_q(q, s2);
        float* ws_slot = direct ? nullptr : a.ws + (size_t)(u + s) * NH * kPartialStride;
        finish<G, KV, NW>(st, lane, wave, direct, a.out + (size_t)s * NH * kHeadDim, ws_slot);
        if (!more) break;
        __syncthreads();  // the next segment's finish rewrites the LDS this one merged from
        s = s2;
        P = P2;
        len = len2;
    }
}

// Head decode for short contexts: workgroup = (query head, sequence), one
// split, NW waves; a step is 8 rows of this head's kv head (256-byte halves of
// the cache rows).  Everything that does not depend on the attended length --
// the query, the new token's k/v and the first DEPTH steps of K/V (rows
// clamped to `bound`, the rows known to be allocated) -- is loaded before the
// length (a device-side position in layer mode) is read, so the position load
// overlaps the K/V traffic.  Every step runs the masked path (rows at or past
// the length get score -inf and V = 0), so the loop carries one copy of the
// softmax state and stale rows past the length never reach the sums.
template <typename T, int G, int KV, int NW, int DEPTH, int MODE>
__device__ __forceinline__ void head_body(const DecodeArgs& a) {
    static_assert(!is_paged(MODE), "the head kernel has no paged modes");
    constexpr int HB = CacheFmt<T>::kHeadBytes;
    constexpr int ROWB = KV * HB;    // cache bytes per row
    constexpr int NH = KV * G;
    constexpr int PPS = kSlots;      // rows per step (one kv head)
    constexpr int STEP = PPS * ROWB;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int head = blockIdx.x, seq = blockIdx.y;
    const int slot = lane / kLanesPerSlot, c = lane % kLanesPerSlot;
    const int kvh = head / G;
    const int lane_colf = kvh * kHeadDim + 4 * c;                     // in fp32 inputs
    const int lane_col = kvh * HB + 4 * c * CacheFmt<T>::kDimBytes;   // in a cache row (bytes)
    const int lane_off = slot * ROWB + lane_col;

    // 1. loads that do not depend on the length
    float q[1][kDimsPerLane];
    load8(q[0], a.q + ((size_t)seq * NH + head) * kHeadDim + 4 * c);
    const RopePrefetch rp = rope_prefetch(a, c);  // (layer mode only: pos_slots is null otherwise)
    float kn[kDimsPerLane], vn[kDimsPerLane];
    const bool new_lane = (MODE == kLayer) && wave == 0 && slot == 0;
    if (new_lane) {
        load8(kn, a.k_new + lane_colf);
        load8(vn, a.v_new + lane_colf);
    }
    size_t base = 0;  // first cache row of the sequence
    int bound;        // rows that may be loaded
    if (MODE == kUniform) {
        base = (size_t)seq * (size_t)a.seq_stride;
        bound = a.n_pos;
    } else if (MODE == kRagged) {
        base = (size_t)a.offsets[seq];
        bound = a.lengths[seq];
    } else {
        bound = a.capacity;
    }
    const char* kb = reinterpret_cast<const char*>(a.k) + base * ROWB + wave * STEP + lane_off;
    const char* vb = reinterpret_cast<const char*>(a.v) + base * ROWB + wave * STEP + lane_off;
    // Byte offset (from kb) of this lane's row in the wave's k-th step, rows
    // clamped below `lim`.
    auto row_off = [&](int k, int lim) {
        const int row = (wave + NW * k) * PPS + slot;
        const int r = min(row, lim - 1);
        return (ptrdiff_t)(r - wave * PPS - slot) * ROWB;
    };
    // Step 0 of every wave is loaded speculatively (rows < bound are allocated);
    // later steps wait for the length so short contexts do not pull the whole
    // allocation through the CU.
    RawRow<T> kbuf[DEPTH], vbuf[DEPTH];
    // (bound >= 1 except for an empty ragged sequence.)
    if (MODE != kRagged || bound > 0) {
        load_raw<T, false>(kbuf[0], kb + row_off(0, bound), c);
        load_raw<T, false>(vbuf[0], vb + row_off(0, bound), c);
    }

    // 2. the attended length
    int n_pos, pos = 0;
    if (MODE == kLayer) {
        pos = a.pos_dev ? *a.pos_dev : a.pos_host;
        if (pos < 0 || pos >= a.capacity || pos >= a.rope_rows) {
            if (head == 0 && threadIdx.x == 0) atomicOr(a.err, 1);
            return;
        }
        n_pos = pos + 1;
    } else {
        n_pos = bound;
    }
    float* out_head = a.out + ((size_t)seq * NH + head) * kHeadDim;
    if (n_pos <= 0) {  // ragged sequence with no rows: defined as a zero output
        if (threadIdx.x < kHeadDim) out_head[threadIdx.x] = 0.f;
        return;
    }
    if (MODE == kRagged && n_pos > a.split_len) {  // longer than the max_len the launch was sized for
        if (threadIdx.x < kHeadDim) out_head[threadIdx.x] = __builtin_nanf("");
        if (threadIdx.x == 0) atomicOr(a.err, 2);
        return;
    }
    const int mem_rows = (MODE == kLayer) ? pos : n_pos;

    // 3. query: RoPE (layer mode) and base-2 softmax scale
    float4 cs0, cs1;
    if (MODE == kLayer) {
        rope_pairs(a, rp, pos, c, cs0, cs1);
        rope8p(q[0], cs0, cs1);
    }
#pragma unroll
    for (int t = 0; t < kDimsPerLane; ++t) q[0][t] *= a.qscale;

    // 4. this wave's steps: wave + NW*k while the step starts below mem_rows
    State<1> st;
    state_init(st);
    const int n_steps = (mem_rows + PPS - 1) / PPS;
    const int nk = (n_steps - wave + NW - 1) / NW;
    // Prefetches are unconditional (rows clamped to the last attended one, an
    // L2 hit past the wave's range), so a 16-bit cache's loads are widened
    // where they are used, not right after a conditional load (which would
    // wait for it on the spot).
    const int lim = max(mem_rows, 1);
#pragma unroll
    for (int d = 1; d < DEPTH; ++d) {
        load_raw<T, false>(kbuf[d], kb + row_off(d, lim), c);
        load_raw<T, false>(vbuf[d], vb + row_off(d, lim), c);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int k0 = 0; k0 < nk; k0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int k = k0 + d;
            if (k < nk) {
                const bool valid = (wave + NW * k) * PPS + slot < mem_rows;
                float kf[kDimsPerLane], vf[kDimsPerLane];
                widen<T>(kf, kbuf[d]);
                widen<T>(vf, vbuf[d]);
#pragma unroll
                for (int t = 0; t < kDimsPerLane; ++t) vf[t] = valid ? vf[t] : 0.f;
                attend<1, 1, true>(q, st, kf, vf, valid);
            }
            load_raw<T, false>(kbuf[d], kb + row_off(k + DEPTH, lim), c);
            load_raw<T, false>(vbuf[d], vb + row_off(k + DEPTH, lim), c);
        }
    }

    // 5. layer mode: the new token (row pos) from registers; its group's first
    //    head writes the rotated k and v to the cache row (tmac_gguf.cpp:1090-1091).
    if (MODE == kLayer && wave == 0) {
        if (new_lane) {
            rope8p(kn, cs0, cs1);
            const bool store = head % G == 0;
            put_row<T>(kn, reinterpret_cast<char*>(a.k_out) + (size_t)pos * ROWB + lane_col, c, store);
            put_row<T>(vn, reinterpret_cast<char*>(a.v_out) + (size_t)pos * ROWB + lane_col, c, store);
        } else {
#pragma unroll
            for (int t = 0; t < kDimsPerLane; ++t) kn[t] = vn[t] = 0.f;
        }
        attend<1, 1, true>(q, st, kn, vn, new_lane);
    }
    finish<1, 1, NW>(st, lane, wave, true, out_head, nullptr);
}

// Sum over all 64 lanes of a wave; every lane receives the same bits (each
// step adds a value and its partner's, which commute exactly).
__device__ __forceinline__ float wave_sum(float x) {
    x = slot_sum(x);     // 8 lanes
    x += dpp<0x140>(x);  // row_mirror: lane i <- lane 15 - i
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Short-context decode with V split over workgroups ("split-V head"
// kernel; fp32 caches).  grid = (query head x VS, sequence), one split.
// Short contexts leave all but a few CUs idle, and each workgroup of the head
// kernel moves its kv head's full K and V half rows (128 KB at 256 rows)
// through one CU, at roughly 80 GB/s per CU.  Here VS workgroups serve one
// query head: each scores all rows (full K) but accumulates only 64/VS dims
// of V, so a CU moves 256 + 256/VS bytes per row instead of 512; the scores
// are computed VS times, from L2.
//   * Lane layout as the head kernel: 8 lanes per row, lane c holds K dims
//     {4c..4c+3, 32+4c..32+4c+3} and DV = 8/VS V dims (vdim0 .. vdim0+DV-1).
//   * Layer mode: the new cache row is rotated and stored right after the
//     position is known, before the rows are attended, so its store latency
//     overlaps the attention; workgroup (head, p) of the group's first head
//     stores V dims of part p, part 0 also the K row.
template <int VS>
__device__ __forceinline__ int hv_vdim0(int vp, int c) {
    return VS == 1 ? 4 * c : VS == 2 ? 32 * vp + 4 * c : VS == 4 ? 16 * vp + 2 * c : 8 * vp + c;
}

template <int DV>
struct VPart {
    float x[DV];
};

template <int VS>
__device__ __forceinline__ void hv_load(VPart<8 / VS>& v, const float* __restrict__ p) {
    if constexpr (VS == 1) {
        const float4 a = *reinterpret_cast<const float4*>(p);
        const float4 b = *reinterpret_cast<const float4*>(p + 32);
        v.x[0] = a.x; v.x[1] = a.y; v.x[2] = a.z; v.x[3] = a.w;
        v.x[4] = b.x; v.x[5] = b.y; v.x[6] = b.z; v.x[7] = b.w;
    } else if constexpr (VS == 2) {
        const float4 a = *reinterpret_cast<const float4*>(p);
        v.x[0] = a.x; v.x[1] = a.y; v.x[2] = a.z; v.x[3] = a.w;
    } else if constexpr (VS == 4) {
        const float2 a = *reinterpret_cast<const float2*>(p);
        v.x[0] = a.x; v.x[1] = a.y;
    } else {
        v.x[0] = *p;
    }
}

template <int VS>
__device__ __forceinline__ void hv_store(float* __restrict__ p, const VPart<8 / VS>& v) {
    if constexpr (VS == 1) {
        *reinterpret_cast<float4*>(p) = make_float4(v.x[0], v.x[1], v.x[2], v.x[3]);
        *reinterpret_cast<float4*>(p + 32) = make_float4(v.x[4], v.x[5], v.x[6], v.x[7]);
    } else if constexpr (VS == 2) {
        *reinterpret_cast<float4*>(p) = make_float4(v.x[0], v.x[1], v.x[2], v.x[3]);
    } else if constexpr (VS == 4) {
        *reinterpret_cast<float2*>(p) = make_float2(v.x[0], v.x[1]);
    } else {
        *p = v.x[0];
    }
}

// V dim t of this lane's part -> position in the head's 64 output dims.
template <int VS>
__device__ __forceinline__ int hv_dim(int vdim0, int t) {
    return VS == 1 ? vdim0 + (t < 4 ? t : 28 + t) : vdim0 + t;
}

template <int G, int KV, int NW, int DEPTH, int MODE, int VS>
__device__ __forceinline__ void hv_body(const DecodeArgs& a) {
    static_assert(MODE == kUniform || MODE == kRagged || MODE == kLayer, "split-V head kernel modes");
    constexpr int DV = 8 / VS;
    constexpr int ROWF = KV * kHeadDim;  // floats per cache row
    constexpr int NH = KV * G;
    constexpr int PPS = kSlots;          // rows per step (one kv head)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // XCD-aware order: XCD x (= blockIdx.x % 8) takes a contiguous run of the
    // logical order (kv head, V part, head in group), so the workgroups that
    // read one kv head's K rows and one V part share an L2.
    const int n_blk = gridDim.x, xcd = blockIdx.x & 7;
    const int per = n_blk >> 3, rem = n_blk & 7;
    const int logical = xcd * per + min(xcd, rem) + (blockIdx.x >> 3);
    const int lt = logical / G;
    const int vp = lt % VS, head = (lt / VS) * G + (logical - lt * G), seq = blockIdx.y;
    const int slot = lane / kLanesPerSlot, c = lane % kLanesPerSlot;
    const int kvh = head / G;
    const int vdim0 = hv_vdim0<VS>(vp, c);

    // 1. loads that do not depend on the length
    float q[1][kDimsPerLane];
    load8(q[0], a.q + ((size_t)seq * NH + head) * kHeadDim + 4 * c);
    const RopePrefetch rp = rope_prefetch(a, c);  // (layer mode only: pos_slots is null otherwise)
    float kn[kDimsPerLane];
    VPart<DV> vn;
    const bool new_lane = (MODE == kLayer) && wave == 0 && slot == 0;
    if (new_lane) {
        load8(kn, a.k_new + kvh * kHeadDim + 4 * c);
        hv_load<VS>(vn, a.v_new + kvh * kHeadDim + vdim0);
    }
    size_t base = 0;
    int bound;
    if (MODE == kUniform) {
        base = (size_t)seq * (size_t)a.seq_stride;
        bound = a.n_pos;
    } else if (MODE == kRagged) {
        base = (size_t)a.offsets[seq];
        bound = a.lengths[seq];
    } else {
        bound = a.capacity;
    }
    const float* kb = a.k + base * ROWF + (size_t)(wave * PPS + slot) * ROWF + kvh * kHeadDim + 4 * c;
    const float* vb = a.v + base * ROWF + (size_t)(wave * PPS + slot) * ROWF + kvh * kHeadDim + vdim0;
    // float offset (from kb / vb) of this lane's row in the wave's k-th step, rows clamped below lim
    auto row_off = [&](int k, int lim) {
        const int row = (wave + NW * k) * PPS + slot;
        const int r = min(row, lim - 1);
        return (ptrdiff_t)(r - wave * PPS - slot) * ROWF;
    };
    float kbuf[DEPTH][kDimsPerLane];
    VPart<DV> vbuf[DEPTH];
    if (MODE != kRagged || bound > 0) {  // step 0 speculatively (rows < bound are allocated)
        load8(kbuf[0], kb + row_off(0, bound));
        hv_load<VS>(vbuf[0], vb + row_off(0, bound));
    }

    // 2. the attended length
    int n_pos, pos = 0;
    if (MODE == kLayer) {
        pos = a.pos_dev ? *a.pos_dev : a.pos_host;
        if (pos < 0 || pos >= a.capacity || pos >= a.rope_rows) {
            if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(a.err, 1);
            return;
        }
        n_pos = pos + 1;
    } else {
        n_pos = bound;
    }
    float* out_head = a.out + ((size_t)seq * NH + head) * kHeadDim;
    if (n_pos <= 0) {  // ragged sequence with no rows: defined as a zero output
        if (threadIdx.x < 8)
            for (int t = 0; t < DV; ++t) out_head[hv_dim<VS>(hv_vdim0<VS>(vp, threadIdx.x), t)] = 0.f;
        return;
    }
    if (MODE == kRagged && n_pos > a.split_len) {  // longer than the max_len the launch was sized for
        if (threadIdx.x < 8)
            for (int t = 0; t < DV; ++t)
                out_head[hv_dim<VS>(hv_vdim0<VS>(vp, threadIdx.x), t)] = __builtin_nanf("");
        if (threadIdx.x == 0) atomicOr(a.err, 2);
        return;
    }
    const int mem_rows = (MODE == kLayer) ? pos : n_pos;
    const int n_steps = (mem_rows + PPS - 1) / PPS;
    const int nk = (n_steps - wave + NW - 1) / NW;
    const int lim = max(mem_rows, 1);
#pragma unroll
    for (int d = 1; d < DEPTH; ++d) {
        load8(kbuf[d], kb + row_off(d, lim));
        hv_load<VS>(vbuf[d], vb + row_off(d, lim));
        __builtin_amdgcn_sched_barrier(0);
    }

    // 3. RoPE (layer mode): q, and the new row, stored now (tmac_gguf.cpp:1090-1091)
    if (MODE == kLayer) {
        float4 t0, t1;
        rope_pairs(a, rp, pos, c, t0, t1);
        rope8p(q[0], t0, t1);
        if (new_lane) {
            rope8p(kn, t0, t1);
            if (head % G == 0) {
                if (vp == 0) store8(a.k_out + (size_t)pos * ROWF + kvh * kHeadDim + 4 * c, kn);
                hv_store<VS>(a.v_out + (size_t)pos * ROWF + kvh * kHeadDim + vdim0, vn);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < kDimsPerLane; ++t) q[0][t] *= a.qscale;

    // 4. this wave's steps: wave + NW*k while the step starts below mem_rows
    float m = kNegInf, l = 0.f, acc[DV];
#pragma unroll
    for (int t = 0; t < DV; ++t) acc[t] = 0.f;
    auto attend_one = [&](const float (&kf)[kDimsPerLane], const VPart<DV>& vf, bool valid) {
        float sc = q[0][0] * kf[0];
#pragma unroll
        for (int t = 1; t < kDimsPerLane; ++t) sc = fmaf(q[0][t], kf[t], sc);
        sc = slot_sum(sc);
        sc = valid ? sc : kNegInf;
        if (__any(sc - m > kTau)) {  // raise the wave's shared max (rare after the first step)
            const float mx = xor_max<kLanesPerSlot>(sc);
            const float mn = fmaxf(m, mx);
            const float alpha = (m == kNegInf) ? 0.f : fast_exp2(m - mn);
            l *= alpha;
#pragma unroll
            for (int t = 0; t < DV; ++t) acc[t] *= alpha;
            m = mn;
        }
        const float e = fast_exp2(sc - m);  // 0 for masked rows
        l += e;
#pragma unroll
        for (int t = 0; t < DV; ++t) acc[t] = fmaf(e, valid ? vf.x[t] : 0.f, acc[t]);
    };
    for (int k0 = 0; k0 < nk; k0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int k = k0 + d;
            if (k < nk) attend_one(kbuf[d], vbuf[d], (wave + NW * k) * PPS + slot < mem_rows);
            load8(kbuf[d], kb + row_off(k + DEPTH, lim));
            hv_load<VS>(vbuf[d], vb + row_off(k + DEPTH, lim));
        }
    }
    // 5. layer mode: the new token (row pos) from registers, by wave 0
    if (MODE == kLayer && wave == 0) {
        if (!new_lane) {
#pragma unroll
            for (int t = 0; t < kDimsPerLane; ++t) kn[t] = 0.f;
#pragma unroll
            for (int t = 0; t < DV; ++t) vn.x[t] = 0.f;
        }
        attend_one(kn, vn, new_lane);
    }

    // 6. slots -> wave total (same max), then waves through LDS
    l = xor_sum<kLanesPerSlot>(l);
#pragma unroll
    for (int t = 0; t < DV; ++t) acc[t] = xor_sum<kLanesPerSlot>(acc[t]);
    __shared__ float s_acc[NW][kLanesPerSlot][DV];
    __shared__ float s_ml[NW][2];
    if (slot == 0) {
#pragma unroll
        for (int t = 0; t < DV; ++t) s_acc[wave][c][t] = acc[t];
        if (c == 0) {
            s_ml[wave][0] = m;
            s_ml[wave][1] = l;
        }
    }
    __syncthreads();
    if (threadIdx.x < kLanesPerSlot * DV) {
        const int cc = threadIdx.x / DV, t = threadIdx.x % DV;
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, s_ml[w][0]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float mw = s_ml[w][0];
            const float sc = (mw == kNegInf) ? 0.f : fast_exp2(mw - M);
            L = fmaf(s_ml[w][1], sc, L);
            A = fmaf(s_acc[w][cc][t], sc, A);
        }
        out_head[hv_dim<VS>(hv_vdim0<VS>(vp, cc), t)] = A / L;
    }
}

// Log-sum-exp merge of the split partials: one wave per (head, sequence) with
// more than one active split, lane d owning output dim d.  Splits go in
// chunks of 32 whose loads are all issued before any is used: lane j loads
// split j's (m, l), every lane its dim of all 32 acc vectors.  The chunk max
// and the l-weighted sum are wave reductions, and split j's weight reaches
// every lane by readlane, so a chunk costs one memory latency; later chunks
// (more than 32 splits) rescale by the running max.
// One chunk of up to 32 partials: lane d's (m, l) of split c0 + d and its dim d
// of every acc vector of the chunk, splits at or past `bound` clamped to the
// last one below it (in bounds; masked by the merge).
constexpr int kMergeChunk = 32;
struct MergeChunk {
    float ml, ll, aj[kMergeChunk];
};
template <int SP>
__device__ __forceinline__ MergeChunk load_chunk(const float* __restrict__ ws, int c0, int bound, int d) {
    MergeChunk ch;
    const int sl = min(c0 + d, bound - 1);
    ch.ml = ws[(size_t)sl * SP + kHeadDim];
    ch.ll = ws[(size_t)sl * SP + kHeadDim + 1];
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) ch.aj[j] = ws[(size_t)min(c0 + j, bound - 1) * SP + d];
    return ch;
}
// Folds the first n splits of a chunk into the running (M, L, A).  Only splits
// j < n enter (a select, so that stale slots past n never reach the sums).
__device__ __forceinline__ void merge_chunk(const MergeChunk& ch, int n, int d, float& M, float& L, float& A) {
    const float mo = d < n ? ch.ml : kNegInf;
    const float cm = xor_max<1>(mo);
    const float nm = fmaxf(M, cm);  // finite: a sequence with rows has a finite score
    const float sc = (M == kNegInf) ? 0.f : fast_exp2(M - nm);
    const float w = (mo == kNegInf) ? 0.f : fast_exp2(mo - nm);
    const float lw = xor_sum<1>(d < n ? ch.ll * w : 0.f);
    float acc = A * sc;
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) {
        const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j));
        acc = j < n ? fmaf(ch.aj[j], wj, acc) : acc;
    }
    A = acc;
    L = fmaf(L, sc, lw);
    M = nm;
}
// Merged value of output dim d over n_act partials, the first at ws (the
// head's partial in that slot) and the rest SP floats apart; `first` is the
// first chunk when the caller loaded it already.
template <int SP>
__device__ __forceinline__ float merge_splits(const float* __restrict__ ws, int n_act, int d,
                                              const MergeChunk* first = nullptr) {
    float M = kNegInf, L = 0.f, A = 0.f;
    for (int c0 = 0; c0 < n_act; c0 += kMergeChunk) {
        const int n = min(kMergeChunk, n_act - c0);
        if (c0 == 0 && first) {
            merge_chunk(*first, n, d, M, L, A);
        } else {
            const MergeChunk ch = load_chunk<SP>(ws, c0, n_act, d);
            merge_chunk(ch, n, d, M, L, A);
        }
    }
    return A / L;
}

template <int G, int KV, int MODE>
__device__ __forceinline__ void combine_body(const DecodeArgs& a) {
    constexpr int NH = KV * G;
    constexpr int SP = NH * kPartialStride;  // floats between splits
    const int h = blockIdx.x, seq = blockIdx.y, d = threadIdx.x;
    // The first chunk's loads go out with the length read: the sequence's
    // n_splits slots are allocated whatever its length (stale slots past its
    // active splits are masked), so one memory latency instead of two.
    const float* ws = a.ws + (size_t)seq * a.n_splits * SP + (size_t)h * kPartialStride;
    const MergeChunk first = load_chunk<SP>(ws, 0, a.n_splits, d);
    int n_pos, pos;
    size_t base;
    if (!seq_geometry<MODE>(a, seq, n_pos, pos, base)) return;
    if (n_pos <= 0) return;
    const int n_act = (n_pos + a.split_len - 1) / a.split_len;
    if (n_act <= 1 || n_act > a.n_splits) return;
    a.out[((size_t)seq * NH + h) * kHeadDim + d] = merge_splits<SP>(ws, n_act, d, &first);
}

// Combine of the stream-K ragged decode: one wave per (head, sequence).  It
// also writes the outputs of the sequences the decode kernel skips: zeros for
// an empty sequence, NaN (and error bit 1) for one longer than max_len.
// LAYER: a position outside the cache or the RoPE table sets error bit 0 and
// leaves the output as it was (as the unit-grid layer kernel does).
template <int G, int KV, bool LAYER>
__device__ __forceinline__ void combine_sk_body(const DecodeArgs& a) {
    constexpr int NH = KV * G;
    constexpr int SP = NH * kPartialStride;
    const int h = blockIdx.x, seq = blockIdx.y, d = threadIdx.x;
    int len;
    if (LAYER) {
        len = sk_len<true>(a, seq);
        if (len == 0) {
            if (h == 0 && d == 0) atomicOr(a.err, 1);
            return;
        }
    } else {
        len = a.lengths[seq];
    }
    float* o = a.out + ((size_t)seq * NH + h) * kHeadDim + d;
    if (len <= 0) {
        *o = 0.f;
        return;
    }
    if (len > a.sk_max_len) {
        *o = __builtin_nanf("");
        if (h == 0 && d == 0) atomicOr(a.err, 2);
        return;
    }
    const int first = a.seg_meta[2 * seq], n_act = a.seg_meta[2 * seq + 1];
    if (n_act <= 1) return;  // written by the decode kernel
    *o = merge_splits<SP>(a.ws + (size_t)first * SP + (size_t)h * kPartialStride, n_act, d);
}

}  // namespace

// Split-V head kernel, V split VS ways (grid x = n_head * VS).
#define TMAC_HV_KERNEL(G, KV, M, MODE, VS)                                                         \
    extern "C" __global__ __launch_bounds__(kHvWaves * 64) void tmac_##M##_hv##VS##_g##G##_kv##KV( \
        DecodeArgs a) {                                                                            \
        hv_body<G, KV, kHvWaves, kHvDepth, MODE, VS>(a);                                  \
    }

#define TMAC_MODE_KERNELS(G, KV, M, MODE)                                                          \
    extern "C" __global__ __launch_bounds__(kGroupWaves * 64) void tmac_##M##_g##G##_kv##KV(        \
        DecodeArgs a) {                                                                            \
        decode_body<float, G, KV, kGroupWaves, kPrefetchDepth, MODE, false>(a);                       \
    }                                                                                              \
    extern "C" __global__ __launch_bounds__(256) void tmac_##M##_g4w_g##G##_kv##KV(DecodeArgs a) {  \
        decode_body<float, G, KV, 4, kPrefetchDepth, MODE, false>(a);                                 \
    }                                                                                              \
    extern "C" __global__ __launch_bounds__(kHeadWaves * 64) void tmac_##M##_head_g##G##_kv##KV(    \
        DecodeArgs a) {                                                                            \
        head_body<float, G, KV, kHeadWaves, kHeadPrefetchDepth, MODE>(a);                           \
    }                                                                                              \
    extern "C" __global__ __launch_bounds__(512) void tmac_##M##_head8_g##G##_kv##KV(DecodeArgs a) { \
        head_body<float, G, KV, 8, kHeadPrefetchDepth, MODE>(a);                                    \
    }                                                                                              \
    extern "C" __global__ __launch_bounds__(256) void tmac_##M##_head4_g##G##_kv##KV(DecodeArgs a) { \
        head_body<float, G, KV, 4, kHeadPrefetchDepth, MODE>(a);                                    \
    }                                                                                              \
    extern "C" __global__ __launch_bounds__(64) void tmac_##M##_combine_g##G##_kv##KV(DecodeArgs a) { \
        combine_body<G, KV, MODE>(a);                                                              \
    }                                                                                              \
    TMAC_HV_KERNEL(G, KV, M, MODE, 1)                                                              \
    TMAC_HV_KERNEL(G, KV, M, MODE, 2)                                                              \
    TMAC_HV_KERNEL(G, KV, M, MODE, 4)                                                              \
    TMAC_HV_KERNEL(G, KV, M, MODE, 8)

// Stream-K ragged decode (fp32 caches) and its combine.
#define TMAC_SK_KERNELS(G, KV)                                                                     \
    extern "C" __global__ __launch_bounds__(256) void tmac_decode_sk_g##G##_kv##KV(DecodeArgs a) {  \
        decode_sk_body<float, G, KV, 4, kPrefetchDepth, false, false>(a);                          \
    }                                                                                              \
    extern "C" __global__ __launch_bounds__(64) void tmac_decode_sk_combine_g##G##_kv##KV(DecodeArgs a) { \
        combine_sk_body<G, KV, false>(a);                                                          \
    }

// Narrow caches (bf16, fp16, Q8_0): the default group (8 waves) and head
// (8 waves) kernels.
#define TMAC_MODE_KERNELS16(G, KV, M, MODE, TN, T, DEPTH)                                              \
    extern "C" __global__ __launch_bounds__(kGroupWaves * 64) void tmac_##M##_##TN##_g##G##_kv##KV(     \
        DecodeArgs a) {                                                                                \
        decode_body<T, G, KV, kGroupWaves, DEPTH, MODE, false>(a);                                     \
    }                                                                                                  \
    extern "C" __global__ __launch_bounds__(512) void tmac_##M##_##TN##_head8_g##G##_kv##KV(DecodeArgs a) { \
        head_body<T, G, KV, 8, kHeadPrefetchDepth, MODE>(a);                                           \
    }

// Paged caches (any element type): decode over block tables, and the batched
// layer step.  Group kernel only (flat unit grid).
#define TMAC_PAGED_KERNELS(G, KV, TN, T, DEPTH)                                                        \
    extern "C" __global__ __launch_bounds__(kGroupWaves * 64) void tmac_decode_p_##TN##_g##G##_kv##KV(  \
        DecodeArgs a) {                                                                                \
        decode_body<T, G, KV, kGroupWaves, DEPTH, kPaged, false>(a);                                   \
    }                                                                                                  \
    extern "C" __global__ __launch_bounds__(kGroupWaves * 64) void tmac_layer_p_##TN##_g##G##_kv##KV(   \
        DecodeArgs a) {                                                                                \
        decode_body<T, G, KV, kGroupWaves, DEPTH, kPagedLayer, false>(a);                              \
    }

// Decode for any shape the compiled kernels do not cover ("any-shape" kernel;
// fp32 caches): runtime n_head, n_kv_head (n_head a multiple of it) and any
// even head_dim up to kAnyMaxDim, as the reference's kernel_attn accepts any
// group and head_dim (kernel_attn.metal:7-60, chosen by attention_op when
// head_dim != 64, metal_backend.hpp:416-452).  grid = (query head, sequence),
// one split, kAnyWaves waves.  A wave step covers 2 rows: lanes 0..31 one
// row, lanes 32..63 the next; lane c of a half holds dims c, c + 32, ...
// (4-byte loads, 128 contiguous bytes per row per load).  q.k is summed over
// the 32 lanes of a half; the online softmax keeps one running max per wave
// (raised when a score exceeds it by kTau); waves merge through LDS.
// Scores use 1/sqrt(head_dim) (tmac_gguf.cpp:1112 for head_dim 64).  Layer
// mode: q and k_new rotated at pos (RoPE pairs (d, d+1) sit in adjacent
// lanes), the group's first head stores row pos, wave 0 attends it.
constexpr int kAnyWaves = kAnyWavesHost;
constexpr int kAnyDpl = kAnyMaxDim / 32;  // dims per lane at most

__device__ __forceinline__ float half_sum(float x) {  // sum over the 32 lanes of a half wave
    x = slot_sum(x);
    x += dpp<0x140>(x);  // row_mirror
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}

__device__ __forceinline__ float other_half(float x) {  // the value of lane l ^ 32
    // The swap returns {lanes 0..31 in both halves, lanes 32..63 in both halves}.
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 32) ? b[0] : b[1]);
}

template <int MODE>
__device__ __forceinline__ void any_body(const DecodeArgs& a) {
    static_assert(MODE == kUniform || MODE == kRagged || MODE == kLayer, "any-shape kernel modes");
    constexpr int NW = kAnyWaves;
    const int hd = a.head_dim, n_head = a.n_head, n_kv = a.n_kv_head;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int half = lane >> 5, c = lane & 31;
    const int head = blockIdx.x, seq = blockIdx.y;
    const int kvh = head / (n_head / n_kv);
    const int ndim = (hd - c + 31) / 32;  // dims of this lane: c + 32 j, j < ndim
    const size_t rowf = (size_t)n_kv * hd;  // floats per cache row

    float q[kAnyDpl];
#pragma unroll
    for (int j = 0; j < kAnyDpl; ++j) q[j] = j < ndim ? a.q[((size_t)seq * n_head + head) * hd + c + 32 * j] : 0.f;
    size_t base = 0;
    int n_pos, pos = 0;
    if (MODE == kUniform) {
        base = (size_t)seq * (size_t)a.seq_stride;
        n_pos = a.n_pos;
    } else if (MODE == kRagged) {
        base = (size_t)a.offsets[seq];
        n_pos = a.lengths[seq];
    } else {
        pos = a.pos_dev ? *a.pos_dev : a.pos_host;
        if (pos < 0 || pos >= a.capacity || pos >= a.rope_rows) {
            if (head == 0 && threadIdx.x == 0) atomicOr(a.err, 1);
            return;
        }
        n_pos = pos + 1;
    }
    n_pos = __builtin_amdgcn_readfirstlane(n_pos);
    pos = __builtin_amdgcn_readfirstlane(pos);
    float* out_head = a.out + ((size_t)seq * n_head + head) * hd;
    if (n_pos <= 0) {
        for (int i = threadIdx.x; i < hd; i += NW * 64) out_head[i] = 0.f;
        return;
    }
    if (MODE == kRagged && n_pos > a.split_len) {
        for (int i = threadIdx.x; i < hd; i += NW * 64) out_head[i] = __builtin_nanf("");
        if (threadIdx.x == 0) atomicOr(a.err, 2);
        return;
    }
    const int mem_rows = MODE == kLayer ? pos : n_pos;
    const float2* cs_row = nullptr;
    if (MODE == kLayer) {  // RoPE of q: the pair partner of dim c + 32 j is lane c ^ 1
        cs_row = a.rope_cs + (size_t)pos * (hd / 2);
#pragma unroll
        for (int j = 0; j < kAnyDpl; ++j) {
            const float xp = dpp<0xB1>(q[j]);
            if (j < ndim) {
                const int d = c + 32 * j;
                const float2 cs = cs_row[d >> 1];
                float x0 = (d & 1) ? xp : q[j], x1 = (d & 1) ? q[j] : xp;
                rotate_pair(x0, x1, cs.x, cs.y);
                q[j] = (d & 1) ? x1 : x0;
            }
        }
    }
    const float qscale = 1.4426950408889634f / sqrtf((float)hd);  // log2(e) / sqrt(head_dim)
#pragma unroll
    for (int j = 0; j < kAnyDpl; ++j) q[j] *= qscale;

    const float* kb = a.k + base * rowf + (size_t)kvh * hd + c;
    const float* vb = a.v + base * rowf + (size_t)kvh * hd + c;
    float m = kNegInf, l = 0.f, acc[kAnyDpl];
#pragma unroll
    for (int j = 0; j < kAnyDpl; ++j) acc[j] = 0.f;
    auto attend_row = [&](const float (&kr)[kAnyDpl], const float (&vr)[kAnyDpl], bool valid) {
        float sc = 0.f;
#pragma unroll
        for (int j = 0; j < kAnyDpl; ++j) sc = fmaf(q[j], kr[j], sc);
        sc = half_sum(sc);
        sc = valid ? sc : kNegInf;
        float mx = fmaxf(sc, other_half(sc));
        if (__any(mx - m > kTau)) {
            const float mn = fmaxf(m, mx);
            const float alpha = (m == kNegInf) ? 0.f : fast_exp2(m - mn);
            l *= alpha;
#pragma unroll
            for (int j = 0; j < kAnyDpl; ++j) acc[j] *= alpha;
            m = mn;
        }
        const float e = fast_exp2(sc - m);
        l += e;
#pragma unroll
        for (int j = 0; j < kAnyDpl; ++j) acc[j] = fmaf(e, valid ? vr[j] : 0.f, acc[j]);
    };
    // wave w takes 2-row steps w, w + NW, ...; two steps of K/V in flight
    const int n_steps = (mem_rows + 1) / 2;
    float k0[kAnyDpl], v0[kAnyDpl], k1[kAnyDpl], v1[kAnyDpl];
    auto load_step = [&](float (&kx)[kAnyDpl], float (&vx)[kAnyDpl], int st) {
        const int r = min(2 * st + half, mem_rows - 1);
#pragma unroll
        for (int j = 0; j < kAnyDpl; ++j) {
            kx[j] = j < ndim ? kb[(size_t)r * rowf + 32 * j] : 0.f;
            vx[j] = j < ndim ? vb[(size_t)r * rowf + 32 * j] : 0.f;
        }
    };
    int st = wave;
    if (st < n_steps) load_step(k0, v0, st);
    for (; st < n_steps; st += 2 * NW) {
        if (st + NW < n_steps) load_step(k1, v1, st + NW);
        attend_row(k0, v0, 2 * st + half < mem_rows);
        if (st + NW >= n_steps) break;
        if (st + 2 * NW < n_steps) load_step(k0, v0, st + 2 * NW);
        attend_row(k1, v1, 2 * (st + NW) + half < mem_rows);
    }
    if (MODE == kLayer && wave == 0) {  // the new token, lanes 0..31
        float kn[kAnyDpl], vn[kAnyDpl];
#pragma unroll
        for (int j = 0; j < kAnyDpl; ++j) {
            kn[j] = j < ndim ? a.k_new[(size_t)kvh * hd + c + 32 * j] : 0.f;
            vn[j] = j < ndim ? a.v_new[(size_t)kvh * hd + c + 32 * j] : 0.f;
            const float xp = dpp<0xB1>(kn[j]);
            if (j < ndim) {
                const int d = c + 32 * j;
                const float2 cs = cs_row[d >> 1];
                float x0 = (d & 1) ? xp : kn[j], x1 = (d & 1) ? kn[j] : xp;
                rotate_pair(x0, x1, cs.x, cs.y);
                kn[j] = (d & 1) ? x1 : x0;
                if (half == 0 && head % (n_head / n_kv) == 0) {
                    a.k_out[(size_t)pos * rowf + (size_t)kvh * hd + d] = kn[j];
                    a.v_out[(size_t)pos * rowf + (size_t)kvh * hd + d] = vn[j];
                }
            }
        }
        attend_row(kn, vn, half == 0);
    }
    // halves -> wave (same max), waves -> LDS
    l += other_half(l);
#pragma unroll
    for (int j = 0; j < kAnyDpl; ++j) acc[j] += other_half(acc[j]);
    __shared__ float s_acc[NW][kAnyMaxDim];
    __shared__ float s_ml[NW][2];
    if (half == 0) {
#pragma unroll
        for (int j = 0; j < kAnyDpl; ++j)
            if (j < ndim) s_acc[wave][c + 32 * j] = acc[j];
        if (c == 0) {
            s_ml[wave][0] = m;
            s_ml[wave][1] = l;
        }
    }
    __syncthreads();
    for (int d = threadIdx.x; d < hd; d += NW * 64) {
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, s_ml[w][0]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float mw = s_ml[w][0];
            const float sc = (mw == kNegInf) ? 0.f : fast_exp2(mw - M);
            L = fmaf(s_ml[w][1], sc, L);
            A = fmaf(s_acc[w][d], sc, A);
        }
        out_head[d] = A / L;
    }
}

#if TMAC_IN_PART(0)
extern "C" __global__ __launch_bounds__(kAnyWaves * 64) void tmac_decode_u_any(DecodeArgs a) { any_body<kUniform>(a); }
extern "C" __global__ __launch_bounds__(kAnyWaves * 64) void tmac_decode_r_any(DecodeArgs a) { any_body<kRagged>(a); }
extern "C" __global__ __launch_bounds__(kAnyWaves * 64) void tmac_layer_any(DecodeArgs a) { any_body<kLayer>(a); }
#endif

#if TMAC_IN_PART(0)
#define TMAC_DECODE_F32(G, KV)                       \
    TMAC_MODE_KERNELS(G, KV, decode_u, kUniform)      \
    TMAC_MODE_KERNELS(G, KV, decode_r, kRagged)       \
    TMAC_MODE_KERNELS(G, KV, layer, kLayer)         \
    TMAC_SK_KERNELS(G, KV)
#else
#define TMAC_DECODE_F32(G, KV)
#endif
#if TMAC_IN_PART(1)
#define TMAC_DECODE_NARROW(G, KV)                                                      \
    TMAC_MODE_KERNELS16(G, KV, decode_u, kUniform, bf16, __bf16, kPrefetchDepth16)      \
    TMAC_MODE_KERNELS16(G, KV, decode_r, kRagged, bf16, __bf16, kPrefetchDepth16)       \
    TMAC_MODE_KERNELS16(G, KV, layer, kLayer, bf16, __bf16, kPrefetchDepth16)           \
    TMAC_MODE_KERNELS16(G, KV, decode_u, kUniform, f16, _Float16, kPrefetchDepth16)     \
    TMAC_MODE_KERNELS16(G, KV, decode_r, kRagged, f16, _Float16, kPrefetchDepth16)      \
    TMAC_MODE_KERNELS16(G, KV, layer, kLayer, f16, _Float16, kPrefetchDepth16)          \
    TMAC_MODE_KERNELS16(G, KV, decode_u, kUniform, q8, q8_0_t, kPrefetchDepthQ8)        \
    TMAC_MODE_KERNELS16(G, KV, decode_r, kRagged, q8, q8_0_t, kPrefetchDepthQ8)         \
    TMAC_MODE_KERNELS16(G, KV, layer, kLayer, q8, q8_0_t, kPrefetchDepthQ8)
#else
#define TMAC_DECODE_NARROW(G, KV)
#endif
#if TMAC_IN_PART(2)
#define TMAC_DECODE_PAGED(G, KV)                                                       \
    TMAC_PAGED_KERNELS(G, KV, f32, float, kPrefetchDepth)                               \
    TMAC_PAGED_KERNELS(G, KV, bf16, __bf16, kPrefetchDepth16)                           \
    TMAC_PAGED_KERNELS(G, KV, f16, _Float16, kPrefetchDepth16)                          \
    TMAC_PAGED_KERNELS(G, KV, q8, q8_0_t, kPrefetchDepthQ8)                             \
    extern "C" __global__ __launch_bounds__(256) void tmac_decode_sk_p_f32_g##G##_kv##KV(DecodeArgs a) { \
        decode_sk_body<float, G, KV, 4, kPrefetchDepth, true, false>(a);                \
    }                                                                                   \
    extern "C" __global__ __launch_bounds__(256) void tmac_layer_sk_p_f32_g##G##_kv##KV(DecodeArgs a) { \
        decode_sk_body<float, G, KV, 4, kPrefetchDepth, true, true>(a);                 \
    }                                                                                   \
    extern "C" __global__ __launch_bounds__(64) void tmac_layer_sk_combine_g##G##_kv##KV(DecodeArgs a) { \
        combine_sk_body<G, KV, true>(a);                                                \
    }                                                                                   \
    extern "C" __global__ __launch_bounds__(64) void tmac_decode_p_combine_g##G##_kv##KV(DecodeArgs a) { \
        combine_body<G, KV, kPaged>(a);                                                 \
    }                                                                                   \
    extern "C" __global__ __launch_bounds__(64) void tmac_layer_p_combine_g##G##_kv##KV(DecodeArgs a) { \
        combine_body<G, KV, kPagedLayer>(a);                                            \
    }
#else
#define TMAC_DECODE_PAGED(G, KV)
#endif
#define TMAC_DECODE_KERNELS(G, KV) TMAC_DECODE_F32(G, KV) TMAC_DECODE_NARROW(G, KV) TMAC_DECODE_PAGED(G, KV)

// (query heads per kv head, kv heads).  Qwen2-0.5B is (7, 2).
TMAC_DECODE_KERNELS(7, 2)
TMAC_DECODE_KERNELS(1, 1)
TMAC_DECODE_KERNELS(1, 2)
TMAC_DECODE_KERNELS(2, 2)
TMAC_DECODE_KERNELS(4, 2)
TMAC_DECODE_KERNELS(4, 4)
TMAC_DECODE_KERNELS(8, 1)

// ---------------------------------------------------------------------------
// Chunked causal prefill on bf16 MFMA (v_mfma_f32_16x16x32_bf16).
//
// Two launches.  The pack kernel rounds the cache rows 0 .. prefix + n_q - 1
// of every (sequence, kv head) to bf16 (nearest even) once, into 64-key tiles
// laid out exactly as the attention kernel keeps them in LDS: K as
// [key][dim], V^T as [dim][key'], 64 x 64 each, 16-byte chunks XOR-swizzled
// per row.  The attention kernel then moves tiles into LDS with direct
// global-to-LDS loads (no registers, no conversion), four tiles per stage,
// double-buffered, one barrier per stage.
//
// Attention workgroup = (16-query block, kv head, sequence), 8 waves.  The
// 1-D grid is ordered so that the blocks of one (sequence, kv head) run on the
// same XCD (workgroups are dealt to the 8 XCDs round-robin) and share its L2
// copy of that head's tiles; within an XCD the longest query blocks start
// first.  Wave w computes tiles 2 * (w / 4) and 2 * (w / 4) + 1 of every stage
// for the query heads 2p and 2p + 1 of the group (p = w % 4; a missing second
// head repeats the first and is not stored), so every K and V^T operand read
// from LDS feeds two heads' MFMAs.  Each wave works transposed,
//   S^T (64 keys x 16 queries) = K (keys x dims) . Q^T         8 MFMAs / head / tile
//   O^T (64 dims x 16 queries) += V^T (dims x keys) . P^T     16 MFMAs / head / tile
// so lane l owns query column l % 16 in every accumulator and the online
// softmax is lane-local except for two lane swaps per tile pair.  The running
// max is only raised when a tile pair exceeds it by more than 2^kTau (a rare,
// wave-uniform branch).  P is split into bf16 hi (truncated) + lo (rounded)
// parts, two PV MFMAs, which keeps the weights to ~2^-16 relative error; with
// bf16-representable q/k/v the result matches an fp32 evaluation to fp32
// rounding.  The two tile halves of a head are merged through LDS at the end.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_void_ptr;

constexpr int kStageElems = kPrefillStageTiles * kPrefillTileElems;  // bf16 per LDS stage buffer (64 KiB)

// Column of key `key` (0..63) in a V^T row.  Inside each 32-key half the
// S^T accumulator hands lane group g4 the keys 4*g4 + i and 16 + 4*g4 + i
// (i < 4); this order puts those 8 keys side by side, so the V^T operand of a
// PV MFMA is one 16-byte read.  The P^T operand uses the same key order.
__device__ __forceinline__ int vt_col(int key) {
    const int k = key & 31;
    return (key & 32) + 8 * ((k & 15) >> 2) + 4 * (k >> 4) + (k & 3);
}
// Inverse of vt_col: the key stored at V^T column p.
__device__ __forceinline__ int vt_key(int p) {
    const int q = p & 31;
    return (p & 32) + 16 * ((q >> 2) & 1) + 4 * (q >> 3) + (q & 3);
}

// Element offset of (row, column) in a 64 x 64 bf16 tile: the 16-byte chunk
// c / 8 of row r is stored at chunk (c / 8) ^ sw(r), sw(r) = (r' ^ r' / 8) % 8
// with r' = r % 16.  An MFMA operand read (16 consecutive rows from a multiple
// of 16, one chunk each) then touches 16 distinct (row parity, chunk) bank
// groups, and the offset of row 16 b + r' is 1024 b plus that of row r'.
__device__ __forceinline__ int tile_offset(int r, int c) {
    const int sw = (r ^ ((r >> 3) & 1)) & 7;
    return r * 64 + ((((c >> 3) ^ sw)) << 3) + (c & 7);
}

__device__ __forceinline__ unsigned bf16_pair(float a, float b) {
    const bf16x2 v = {(__bf16)a, (__bf16)b};  // round to nearest even
    return __builtin_bit_cast(unsigned, v);
}

// Max / sum over the four lanes l % 16 + 16 * k (k = 0..3) of a wave, via the
// gfx950 row and half-wave swaps (each returns both swapped registers; the
// reduction of the pair is the same whichever way round they come).
__device__ __forceinline__ float max4_rows(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum4_rows(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Pack one 64-row tile of one (sequence, kv head) from a cache of element
// type T (fp32, bf16, fp16 or Q8_0 head rows), contiguous or paged: 256
// threads, thread t owns row t / 4 and the 8-dim chunks q4 and 4 + q4
// (q4 = t % 4) of the K tile and of the V^T tile.  Values are widened exactly
// to fp32 (load_row) and rounded to bf16 (nearest even; exact for a bf16
// cache).  Only rows row_lo .. n_rows - 1 are written: the other rows of a
// tile keep what an earlier pack left there (the attention kernel reads no
// row past the last query's key, so rows never packed may hold anything).
// A launch packs the tiles tile0 .. tile0 + n_tpp - 1 of every (sequence,
// kv head).
template <typename T, int KV, bool PAGED>
__device__ __forceinline__ void prefill_pack_body(const PrefillArgs& a) {
    constexpr int HB = CacheFmt<T>::kHeadBytes, ROWB = KV * HB, DB = CacheFmt<T>::kDimBytes;
    const int tile = a.tile0 + blockIdx.x % a.n_tpp;
    const int rest = blockIdx.x / a.n_tpp;
    const int kv = rest % KV, seq = rest / KV;
    const int tid = threadIdx.x, r = tid >> 2, q4 = tid & 3;
    const int key = tile * kPrefillKeys + r;
    const int kr = min(key, a.n_rows - 1);
    size_t row;
    if constexpr (PAGED) {
        int pg = a.block_table[(size_t)seq * a.max_pages + (kr >> kPageShift)];
        if (pg < 0 || pg >= a.n_pages) {  // clamped into the pool, reported
            if (key < a.n_rows && (key & (kPageRows - 1)) == 0 && q4 == 0) atomicOr(a.err, 4);  // once per page
            pg = min(max(pg, 0), a.n_pages - 1);
        }
        row = (size_t)pg * kPageRows + (kr & (kPageRows - 1));
    } else {
        row = (size_t)seq * a.seq_stride + (size_t)kr;
    }
    const char* kh = reinterpret_cast<const char*>(a.k) + row * ROWB + kv * HB;
    const char* vh = reinterpret_cast<const char*>(a.v) + row * ROWB + kv * HB;
    const bool valid = key >= a.row_lo && key < a.n_rows;
    __shared__ float sv[64][65];
    // load_row(c) gives dims 4c..4c+3 and 32+4c..32+4c+3; c = 2 q4 and 2 q4 + 1
    // together hold the chunks 8 q4 .. 8 q4 + 7 and 32 + 8 q4 .. 32 + 8 q4 + 7.
    float k0[8], k1[8], v0[8], v1[8];
    load_row<T, false>(k0, kh + 4 * (2 * q4) * DB, 2 * q4);
    load_row<T, false>(k1, kh + 4 * (2 * q4 + 1) * DB, 2 * q4 + 1);
    load_row<T, false>(v0, vh + 4 * (2 * q4) * DB, 2 * q4);
    load_row<T, false>(v1, vh + 4 * (2 * q4 + 1) * DB, 2 * q4 + 1);
    float kx[2][8];  // [chunk: 8 q4.., 32 + 8 q4..][dim]
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        kx[0][t] = valid ? k0[t] : 0.f;
        kx[0][4 + t] = valid ? k1[t] : 0.f;
        kx[1][t] = valid ? k0[4 + t] : 0.f;
        kx[1][4 + t] = valid ? k1[4 + t] : 0.f;
        sv[r][8 * q4 + t] = valid ? v0[t] : 0.f;
        sv[r][8 * q4 + 4 + t] = valid ? v1[t] : 0.f;
        sv[r][32 + 8 * q4 + t] = valid ? v0[4 + t] : 0.f;
        sv[r][32 + 8 * q4 + 4 + t] = valid ? v1[4 + t] : 0.f;
    }
    __bf16* dst = reinterpret_cast<__bf16*>(a.packed) +
                  (((size_t)seq * KV + kv) * a.n_tp + tile) * kPrefillTileElems;
    if (valid) {
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const float* x = kx[cc];
            const u32x4 w = {bf16_pair(x[0], x[1]), bf16_pair(x[2], x[3]), bf16_pair(x[4], x[5]),
                             bf16_pair(x[6], x[7])};
            *reinterpret_cast<u32x4*>(dst + tile_offset(r, 32 * cc + 8 * q4)) = w;
        }
    }
    __syncthreads();
    // V^T row d = r, columns p = 16 * q4 .. + 15 hold keys vt_key(p).  A chunk
    // whose 8 keys straddle row_lo or n_rows keeps the old values of the keys
    // outside (read back and merged per 16-bit element).
    const int tkey0 = tile * kPrefillKeys;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
        float x[8];
        unsigned keep = 0;  // bit e: key e of the chunk lies outside row_lo .. n_rows - 1
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int kk = vt_key(16 * q4 + 8 * cc + e);
            x[e] = sv[kk][r];
            keep |= (tkey0 + kk < a.row_lo || tkey0 + kk >= a.n_rows) ? 1u << e : 0u;
        }
        u32x4 w = {bf16_pair(x[0], x[1]), bf16_pair(x[2], x[3]), bf16_pair(x[4], x[5]), bf16_pair(x[6], x[7])};
        u32x4* p = reinterpret_cast<u32x4*>(dst + 64 * 64 + tile_offset(r, 16 * q4 + 8 * cc));
        if (keep == 0xFFu) continue;
        if (keep) {
            const u32x4 old = *p;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const unsigned mk = ((keep >> (2 * i)) & 1u ? 0x0000FFFFu : 0u) |
                                    ((keep >> (2 * i + 1)) & 1u ? 0xFFFF0000u : 0u);
                w[i] = (w[i] & ~mk) | (old[i] & mk);
            }
        }
        *p = w;
    }
}

template <int G, int KV>
__device__ __forceinline__ void prefill_body(const PrefillArgs& a) {
    constexpr int NH = KV * G;
    constexpr int QB = kPrefillQueries, KT = kPrefillKeys, NT = kPrefillStageTiles;
    static_assert(G <= 2 * 4, "four head pairs per workgroup");
    static_assert(kPrefillWaves == 2 * NT, "one wave per (head pair, half stage)");
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pair = wave & 3, part = wave >> 2;  // head pair, half of the stage (two tiles)

    // XCD-aware block order: XCD x (= blockIdx.x % 8) owns a contiguous run of
    // the logical block range.
    const int n_blk = gridDim.x, xcd = blockIdx.x & 7;
    const int per = n_blk >> 3, rem = n_blk & 7;
    const int logical = xcd * per + min(xcd, rem) + (blockIdx.x >> 3);
    const int sk = logical / a.n_qblk;                  // (sequence, kv head)
    const int qblk = a.n_qblk - 1 - (logical - sk * a.n_qblk);
    const int seq = sk / KV, kv = sk - seq * KV;
    const int q0 = qblk * QB;
    const int q_last = min(q0 + QB, a.n_q) - 1;
    const int kmax = a.prefix_len + q_last;  // last key any query of the block attends
    const int n_tiles = kmax / KT + 1;
    const int n_stages = (n_tiles + NT - 1) / NT;
    const __bf16* slab = reinterpret_cast<const __bf16*>(a.packed) + (size_t)sk * a.n_tp * kPrefillTileElems;

    // Two stage buffers as separate objects, so that the compiler sees that a
    // direct load into one does not alias the operand reads from the other.
    __shared__ __attribute__((aligned(16))) __bf16 buf0[kStageElems];
    __shared__ __attribute__((aligned(16))) __bf16 buf1[kStageElems];

    const int col = lane & 15;  // query column / MFMA row index
    const int g4 = lane >> 4;   // k-group of the MFMA operands
    const bool compute = 2 * pair < G;
    const int hl[2] = {min(2 * pair, G - 1), min(2 * pair + 1, G - 1)};
    const int qi = q0 + col;
    const int ap = a.prefix_len + qi;  // absolute position of this lane's query
    const float c = a.qscale;

    // Q^T operands: this lane's query, dims 32j + 8*g4 + (0..7).
    bf16x8 qop[2][2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const float* qp = a.q + (((size_t)seq * a.n_q + min(qi, a.n_q - 1)) * NH + kv * G + hl[hh]) * kHeadDim;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float4 x0 = *reinterpret_cast<const float4*>(qp + 32 * j + 8 * g4);
            const float4 x1 = *reinterpret_cast<const float4*>(qp + 32 * j + 8 * g4 + 4);
            const u32x4 w = {bf16_pair(x0.x, x0.y), bf16_pair(x0.z, x0.w), bf16_pair(x1.x, x1.y),
                             bf16_pair(x1.z, x1.w)};
            qop[hh][j] = __builtin_bit_cast(bf16x8, w);
        }
    }
    // per-lane operand offsets inside a K or V^T tile: rows 16 b + col, chunk 4 j + g4
    int op_off[4][2];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int j = 0; j < 2; ++j) op_off[b][j] = tile_offset(16 * b + col, 32 * j + 8 * g4);

    // O^T blocks 0..3: dims 16*db + 4*g4 + i for query col.  Block 4 is the
    // softmax row sum: its A operand is a constant row of ones (row 0 of the
    // block), so O^T[4] row 0 = sum over keys of P, accumulated from the same
    // bf16 hi/lo weights as the output.
    f32x4 o[2][5];
    float m[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        m[hh] = kNegInf;
#pragma unroll
        for (int db = 0; db < 5; ++db) o[hh][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = (__bf16)(col == 0 ? 1.f : 0.f);

    // Direct loads of stage st (NT tiles, contiguous in the slab): each wave
    // moves kPieces KiB; lane l's 16 bytes land at piece + 16 l.
    constexpr int kPieces = kStageElems / 512 / kPrefillWaves;
    auto dma = [&](int st, __bf16* dst) {
        const __bf16* src = slab + (size_t)st * kStageElems + (wave * kPieces) * 512 + lane * 8;
#pragma unroll
        for (int i = 0; i < kPieces; ++i)
            __builtin_amdgcn_global_load_lds(src + i * 512, (lds_void_ptr)(dst + (wave * kPieces + i) * 512), 16,
                                             0, 0);
    };

    // Two consecutive tiles (keys kbase .. kbase + 127) for the wave's two
    // heads; `diag` (wave-uniform) applies the causal mask.
    auto tile_pair = [&](const __bf16* tb, int kbase, bool diag) {
        f32x4 sc[2][2][4];  // [tile][head][key block]
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const __bf16* tk = tb + u * kPrefillTileElems;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                sc[u][0][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
                sc[u][1][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const bf16x8 ka = *reinterpret_cast<const bf16x8*>(tk + op_off[kb][j]);
                    sc[u][0][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qop[0][j], sc[u][0][kb], 0, 0, 0);
                    sc[u][1][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qop[1][j], sc[u][1][kb], 0, 0, 0);
                }
            }
        }
        if (diag) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int lim = ap - kbase - KT * u - 4 * g4;  // key 16 kb + i of tile u is visible iff <= lim
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (16 * kb + i > lim) sc[u][hh][kb][i] = kNegInf;
            }
        }
        float tm[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            tm[hh] = kNegInf;
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) tm[hh] = fmaxf(tm[hh], sc[u][hh][kb][i]);
            tm[hh] = max4_rows(tm[hh]);
        }
        // raise a running max only when the pair exceeds it by > 2^kTau (rare, wave-uniform)
        if (__any((tm[0] - m[0]) * c > kTau || (tm[1] - m[1]) * c > kTau)) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const float mn = fmaxf(m[hh], tm[hh]);
                const float alpha = (m[hh] == kNegInf) ? 0.f : fast_exp2((m[hh] - mn) * c);
                m[hh] = mn;
#pragma unroll
                for (int db = 0; db < 5; ++db) o[hh][db] *= alpha;
            }
        }
        const float mc[2] = {(m[0] == kNegInf) ? 0.f : m[0] * c, (m[1] == kNegInf) ? 0.f : m[1] * c};
        // P^T (hi, lo) and O^T += V^T . P^T; one basic block, so exponentials
        // of one (tile, head) can issue under the MFMAs of the previous one.
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const __bf16* tv = tb + u * kPrefillTileElems + 64 * 64;
            bf16x8 va[4][2];
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int j = 0; j < 2; ++j) va[db][j] = *reinterpret_cast<const bf16x8*>(tv + op_off[db][j]);
            // Keys past the block's last query are rows a pack need not have
            // written: their weights are 0, and their V is set to 0 so that no
            // NaN or infinity left there reaches the product.
            const int vlim = kmax - kbase - KT * u;  // keys of tile u above vlim (wave-uniform)
            if (diag && vlim < KT - 1) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    u32x4 keep;
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        const int p0 = 32 * j + 8 * g4 + 2 * w;
                        keep[w] = (vt_key(p0) <= vlim ? 0x0000FFFFu : 0u) | (vt_key(p0 + 1) <= vlim ? 0xFFFF0000u : 0u);
                    }
#pragma unroll
                    for (int db = 0; db < 4; ++db)
                        va[db][j] = __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4, va[db][j]) & keep);
                }
            }
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                // P^T operands for PV K-step j: keys 32j + 16h + 4*g4 + i  <->  S^T block 2j + h, row i
                u32x4 ph[2], pl[2];
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
#pragma unroll
                        for (int i = 0; i < 4; i += 2) {
                            const float p0 = fast_exp2(__builtin_fmaf(sc[u][hh][2 * j + h][i], c, -mc[hh]));
                            const float p1 = fast_exp2(__builtin_fmaf(sc[u][hh][2 * j + h][i + 1], c, -mc[hh]));
                            const unsigned u0 = __float_as_uint(p0) & 0xffff0000u;
                            const unsigned u1 = __float_as_uint(p1) & 0xffff0000u;
                            ph[j][2 * h + i / 2] = (u0 >> 16) | u1;
                            pl[j][2 * h + i / 2] =
                                bf16_pair(p0 - __uint_as_float(u0), p1 - __uint_as_float(u1));
                        }
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        o[hh][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            va[db][j], __builtin_bit_cast(bf16x8, ph[j]), o[hh][db], 0, 0, 0);
                        o[hh][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            va[db][j], __builtin_bit_cast(bf16x8, pl[j]), o[hh][db], 0, 0, 0);
                    }
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    o[hh][4] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, __builtin_bit_cast(bf16x8, ph[j]),
                                                                       o[hh][4], 0, 0, 0);
                    o[hh][4] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, __builtin_bit_cast(bf16x8, pl[j]),
                                                                       o[hh][4], 0, 0, 0);
                }
            }
        }
    };

    // Stage st: start the direct loads of stage st + 1 into the other buffer
    // (last read before the previous barrier), compute this wave's two tiles,
    // then wait for this wave's loads and meet at the barrier.  Every stage
    // holds NT tiles of the slab (n_tp is a multiple of NT); tiles past the
    // block's last key are masked entirely (their keys exceed every query).
    const int diag_from = a.prefix_len + q0 - (2 * KT - 1);  // tile pairs at or after this key need the mask
    auto stage = [&](int st, const __bf16* cur, __bf16* nxt) {
        if (st + 1 < n_stages) dma(st + 1, nxt);
        const int ta = NT * st + 2 * part;
        if (compute && ta < n_tiles) tile_pair(cur + 2 * part * kPrefillTileElems, ta * KT, ta * KT > diag_from);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's direct loads have landed
        __syncthreads();
    };

    dma(0, buf0);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    for (int st = 0; st < n_stages; st += 2) {
        stage(st, buf0, buf1);
        if (st + 1 < n_stages) stage(st + 1, buf1, buf0);
    }

    // Merge the two stage halves of each head: part 1 hands (m, l, O) to part 0
    // through LDS (the stage buffers are free after the last barrier).  Pairs
    // 0-1 use buf0, pairs 2-3 buf1: [pair % 2][head][18][64] floats.
    static_assert(2 * 2 * 18 * 64 * 4 <= kStageElems * 2, "merge areas fit the stage buffers");
    float* mgp = reinterpret_cast<float*>(pair < 2 ? buf0 : buf1) + (pair & 1) * 2 * 18 * 64;
    float l[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) l[hh] = sum4_rows(g4 == 0 ? o[hh][4][0] : 0.f);
    if (compute && part > 0) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            float* dst = mgp + hh * 18 * 64 + lane;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[(4 * db + i) * 64] = o[hh][db][i];
            dst[16 * 64] = m[hh];
            dst[17 * 64] = l[hh];
        }
    }
    __syncthreads();
    if (!compute || part > 0 || qi >= a.n_q) return;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        if (hh == 1 && 2 * pair + 1 >= G) break;
        const float* src = mgp + hh * 18 * 64 + lane;
        const float m1 = src[16 * 64], l1 = src[17 * 64];
        const float mx = fmaxf(m[hh], m1);  // m[hh] is finite: part 0 holds tile 0, whose key 0 every query sees
        const float a0 = fast_exp2((m[hh] - mx) * c);
        const float a1 = (m1 == kNegInf) ? 0.f : fast_exp2((m1 - mx) * c);
        const float inv = 1.f / (a0 * l[hh] + a1 * l1);
        float* op = a.out + (((size_t)seq * a.n_q + qi) * NH + kv * G + hl[hh]) * kHeadDim + 4 * g4;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            float4 r;
            r.x = (a0 * o[hh][db][0] + a1 * src[(4 * db + 0) * 64]) * inv;
            r.y = (a0 * o[hh][db][1] + a1 * src[(4 * db + 1) * 64]) * inv;
            r.z = (a0 * o[hh][db][2] + a1 * src[(4 * db + 2) * 64]) * inv;
            r.w = (a0 * o[hh][db][3] + a1 * src[(4 * db + 3) * 64]) * inv;
            *reinterpret_cast<float4*>(op + 16 * db) = r;
        }
    }
}

#define TMAC_PREFILL_KERNEL(G, KV)                                                                    \
    extern "C" __global__ __launch_bounds__(kPrefillWaves * 64) void tmac_prefill_g##G##_kv##KV(      \
        PrefillArgs a) {                                                                              \
        prefill_body<G, KV>(a);                                                                       \
    }
#if TMAC_IN_PART(3)
TMAC_PREFILL_KERNEL(7, 2)
TMAC_PREFILL_KERNEL(1, 1)
TMAC_PREFILL_KERNEL(1, 2)
TMAC_PREFILL_KERNEL(2, 2)
TMAC_PREFILL_KERNEL(4, 2)
TMAC_PREFILL_KERNEL(4, 4)
TMAC_PREFILL_KERNEL(8, 1)

#define TMAC_PREFILL_PACK_TYPE(KV, TN, T)                                                                  \
    extern "C" __global__ __launch_bounds__(256) void tmac_prefill_pack_##TN##kv##KV(PrefillArgs a) {      \
        prefill_pack_body<T, KV, false>(a);                                                               \
    }                                                                                                      \
    extern "C" __global__ __launch_bounds__(256) void tmac_prefill_pack_p_##TN##kv##KV(PrefillArgs a) {    \
        prefill_pack_body<T, KV, true>(a);                                                                \
    }
#define TMAC_PREFILL_PACK_KERNEL(KV)            \
    TMAC_PREFILL_PACK_TYPE(KV, , float)         \
    TMAC_PREFILL_PACK_TYPE(KV, bf16_, __bf16)   \
    TMAC_PREFILL_PACK_TYPE(KV, f16_, _Float16)  \
    TMAC_PREFILL_PACK_TYPE(KV, q8_, q8_0_t)
TMAC_PREFILL_PACK_KERNEL(1)
TMAC_PREFILL_PACK_KERNEL(2)
TMAC_PREFILL_PACK_KERNEL(4)
#endif

// ---------------------------------------------------------------------------
// Decode on MFMA for bf16 caches (v_mfma_f32_16x16x32_bf16 for q.k,
// v_mfma_f32_16x16x16_bf16 for p.v).  The VALU group kernel spends ~20
// instructions per (row, query head) whatever the row's bytes, so a bf16 cache
// would be VALU-bound there; here the products run on the matrix cores and
// the VALU only does the softmax, four values per lane per 16-row tile.
//
// Same workgroups as the group kernel: grid (split, sequence) or the flat unit
// grid, 8 waves, the same splits, combine and page addressing.  In the layer
// modes the query is rotated before it is split, and the new token (RoPE,
// rounding to the cache type and the cache write exactly as the VALU kernels
// do them) is attended as one more partial in the merge.  Wave w takes
// the 16-row tiles w, w + 8, ... of its range.  Per tile (16 positions):
//   S^T (16 keys x 16 columns) = K (16 x KV*64) . Qbd^T.  Column c < n_head is
//     query head c; Qbd is block diagonal, so column c only meets the 64 dims
//     of its own kv head.  The pre-scaled fp32 query is split into three
//     bf16 parts (hi + mid + lo, 2^-27 relative), three MFMAs per 32 dims: a
//     two-part split (2^-18) left score errors of ~2e-4 with keys 8x larger
//     than the query, outside the fp32 contract.
//   P^T = exp2(S^T - m), online, with the lazy rescale of the VALU kernel; P
//     is split into bf16 hi (truncated) + lo (nearest) before the p.v MFMAs.
//   O^T (KV*64 dims x 16 columns) += V^T . P^T over KV*4 blocks of 16 dims.
//     The V tile is copied to LDS (rows of the cache, 16-byte chunks
//     XOR-swizzled per row) and read back with ds_read_b64_tr_b16: in each
//     group of 16 lanes, lane 4e + j/4 ... fetches 8 bytes and lane i receives
//     element i % 4 of lane 4e + i / 4's 8 bytes, so lane j pointing at row
//     4g + j/4, dims 16b + 4(j % 4) hands every lane 4 consecutive keys of one
//     dim: the V^T operand, with no VALU transposition.
// In the S^T / P^T / O^T accumulators lane l holds column l % 16 and rows
// 4 (l / 16) + 0..3, so P^T feeds the p.v MFMA from the same registers.
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_v;
typedef __attribute__((address_space(3))) bf16x4_v* lds_bf16x4_ptr;
typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 f16x4_v;
typedef __attribute__((address_space(3))) f16x4_v* lds_f16x4_ptr;

// The 16-bit element types of the MFMA decode: operand types, the matching
// MFMAs and transposed LDS read, and packing of fp32 pairs (nearest even).
//   bf16: fp32's exponent range, so q and P are split as they are.
//   fp16: q is scaled per column by a power of two (its largest |value| to
//   [2^14, 2^15)) and P by 2^7 before splitting, so the split parts stay in
//   fp16's normal range; both scales are undone exactly after the MFMAs.
template <typename T>
struct MMath;
template <>
struct MMath<__bf16> {
    typedef bf16x8 v8;
    typedef i16x4 v4;
    static constexpr bool kScaleQ = false;
    static constexpr int kQParts = 3;  // 16-bit parts of an fp32 query element
    static constexpr float kPScale = 1.0f;
    __device__ static unsigned pack2(float a, float b) { return bf16_pair(a, b); }
    __device__ static float lo(unsigned w) { return __uint_as_float(w << 16); }
    __device__ static float hi(unsigned w) { return __uint_as_float(w & 0xffff0000u); }
    __device__ static f32x4 mfma32(v8 a, v8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
    __device__ static v8 cat(v4 a, v4 b) { return __builtin_bit_cast(v8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7)); }
    __device__ static v4 read_tr(char* p) {
        return __builtin_bit_cast(v4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_ptr)p));
    }
};
template <>
struct MMath<_Float16> {
    typedef f16x8 v8;
    typedef f16x4 v4;
    static constexpr bool kScaleQ = true;
    static constexpr int kQParts = 2;
    static constexpr float kPScale = 128.0f;
    __device__ static unsigned pack2(float a, float b) {
        const f16x2 v = {(_Float16)a, (_Float16)b};
        return __builtin_bit_cast(unsigned, v);
    }
    __device__ static float lo(unsigned w) { return half_bits_to_float(w & 0xffffu); }
    __device__ static float hi(unsigned w) { return half_bits_to_float(w >> 16); }
    __device__ static f32x4 mfma32(v8 a, v8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
    __device__ static v8 cat(v4 a, v4 b) { return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7); }
    __device__ static v4 read_tr(char* p) {
        return __builtin_bit_cast(v4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_f16x4_ptr)p));
    }
};

constexpr int kMTileRows = 16;  // positions per tile
// Waves per workgroup.  bf16 / fp16 caches: 4 (each wave streams twice the
// rows and the final merge halves: config 3 77.7 vs 79.1 us at 8).  Q8_0
// caches: 8, two waves per SIMD hiding each other's widening and LDS
// latency (52 vs 58 us at 4).
template <typename T>
constexpr int mdecode_waves() {
    return __is_same(T, q8_0_t) ? kMWavesQ8Host : kMWaves16Host;
}
// Tiles of K and V in flight per wave.  With the tile loop's exact waits, 2
// beats 3 (3 spills registers for Q8_0 and fp16 caches, and was 0.5% slower
// for bf16 at config 3).
constexpr int kMDepth = 2;

template <typename T, int KV>
struct MTile {
    static constexpr int ROWB = KV * kHeadDim * 2;   // bytes per cache row (16-bit elements)
    static constexpr int CPR = ROWB / 16;            // 16-byte chunks per row
    static constexpr int NV = kMTileRows * CPR / 64; // V chunks per lane per tile
    static constexpr int NKB = 2 * KV;               // 32-dim blocks of the q.k contraction
    static constexpr int NMB = 4 * KV;               // 16-dim blocks of the output
    typename MMath<T>::v8 k[NKB];
    u32x4 v[NV];
};

template <int KV>
__device__ __forceinline__ int mswz(int r) {  // chunk XOR of row r in the LDS copy
    return (2 * r) & (MTile<__bf16, KV>::CPR - 1);
}

// Loads one tile: rows `row0 + 0..15` at `base` (the tile's row 0), rows at or
// past `valid` replaced by row valid - 1 (in bounds, masked later).  A K
// operand load covers 64 bytes of each of 16 rows, so every 128-byte line is
// read by two consecutive loads: K uses normal loads, which keep the line in
// L2 for the second one (non-temporal K loads re-fetched part of those lines
// from HBM: 1.058x the algorithmic bytes against 1.025x, 97 vs 86 us at
// config 3).  V rows are read whole, 1 KB per load, and stay non-temporal.
template <typename T, int KV>
__device__ __forceinline__ void mtile_load(MTile<T, KV>& t, const char* __restrict__ kbase,
                                           const char* __restrict__ vbase, int valid, int lane) {
    using Tile = MTile<T, KV>;
    typedef typename MMath<T>::v8 v8;
    constexpr int ROWB = Tile::ROWB, CPR = Tile::CPR;
    const int col = lane & 15, g = lane >> 4;
    const int kr = min(col, valid - 1);
#pragma unroll
    for (int b = 0; b < Tile::NKB; ++b)
        t.k[b] = *reinterpret_cast<const v8*>(kbase + kr * ROWB + 64 * b + 16 * g);
#pragma unroll
    for (int i = 0; i < Tile::NV; ++i) {
        const int q = 64 * i + lane, r = min(q / CPR, valid - 1), c = q % CPR;
        t.v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vbase + r * ROWB + 16 * c));
    }
}

// Q8_0 caches on the bf16 MFMAs: an int8 value is exact in bf16 and bf16
// has fp32's exponent range, so P times the per-key V scale needs no
// rescaling.  A 16-row tile of 68-byte head rows is one contiguous run of
// 16 * KV * 68 bytes: it is loaded as aligned 16-byte chunks (head rows are
// only 4-byte aligned, so per-operand loads would be misaligned and many),
// staged raw in LDS, and the K operands, scales and V runs are read from
// there; V is widened to bf16 into the 16-bit V tile layout above.
template <int KV>
struct MTileQ8 {
    static constexpr int ROWB = KV * kQ8HeadBytes;  // cache bytes per row
    static constexpr int RAW = kMTileRows * ROWB;   // bytes per tensor tile
    static constexpr int NCH = RAW / 16;            // 16-byte chunks per tensor tile
    static constexpr int NF = NCH / 64;             // chunk loads per lane and tensor covering 64 chunks
    static constexpr int REM = NCH % 64;            // chunks left per tensor: K's and V's share one load
    static_assert(NF >= 1 && REM > 0 && 2 * REM <= 64, "68-byte head rows: 16 KV rows of 4-byte words");
    static constexpr int NKB = 2 * KV;
    static constexpr int NMB = 4 * KV;
    static constexpr int NVU = kMTileRows * KV * 4 / 64;  // 16-value V runs per lane per tile
    u32x4 k[NF], v[NF];
    u32x4 x;  // lane e < REM: K chunk 64 NF + e; REM <= e < 2 REM: V chunk 64 NF + e - REM
};

// Lane `lane`'s chunk of the shared remainder load: (tensor is V, chunk index).
template <int KV>
__device__ __forceinline__ int2 q8_rem_chunk(int lane) {
    using Tile = MTileQ8<KV>;
    const int e = lane % (2 * Tile::REM);  // lanes past 2 REM repeat the first 2 REM (same lines)
    return int2{e >= Tile::REM, 64 * Tile::NF + e % Tile::REM};
}

// A full tile: chunks 64 i + lane of each tensor, then the K and V remainders
// in one load.  K chunks use normal loads (a tile's first and last 128-byte
// lines are shared with the neighbouring tiles, which other waves read at
// about the same time: 77 -> 73 us at config 3), V chunks non-temporal loads.
template <int KV>
__device__ __forceinline__ void mtile_load_q8(MTileQ8<KV>& t, const char* __restrict__ kbase,
                                              const char* __restrict__ vbase, int lane) {
    using Tile = MTileQ8<KV>;
#pragma unroll
    for (int i = 0; i < Tile::NF; ++i) {
        t.k[i] = *reinterpret_cast<const u32x4*>(kbase + 16 * (64 * i + lane));  // normal: see mtile_load
        t.v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vbase + 16 * (64 * i + lane)));
    }
    const int2 rc = q8_rem_chunk<KV>(lane);
    t.x = *reinterpret_cast<const u32x4*>((rc.x ? vbase : kbase) + 16 * rc.y);
}

// A partial tile (valid < 16 rows) straight into the LDS raw areas, word by
// word, reading only the valid rows' bytes.
template <int KV>
__device__ __forceinline__ void mtile_tail_q8(const char* __restrict__ kbase, const char* __restrict__ vbase,
                                              int valid, char* rk, char* rv, int lane) {
    using Tile = MTileQ8<KV>;
    const int n4 = valid * Tile::ROWB / 4;
#pragma unroll
    for (int i = 0; i < (Tile::RAW / 4 + 63) / 64; ++i) {
        const int w = 64 * i + lane;
        if (w < n4) {
            reinterpret_cast<unsigned*>(rk)[w] = reinterpret_cast<const unsigned*>(kbase)[w];
            reinterpret_cast<unsigned*>(rv)[w] = reinterpret_cast<const unsigned*>(vbase)[w];
        }
    }
}

// Four int8 (one word) -> four bf16 (two words, element 2i in the low half), exactly.
__device__ __forceinline__ u32x2 i8x4_to_bf16(unsigned w) {
    const float f0 = (float)(signed char)w, f1 = (float)(signed char)(w >> 8);
    const float f2 = (float)(signed char)(w >> 16), f3 = (float)(signed char)(w >> 24);
    return u32x2{__builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u),
                 __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u)};
}

// Four int8 (one word) -> four fp16 (two words, element 2i in the low half),
// exactly: byte b becomes u = b ^ 0x80 = b + 128, the fp16 with bits
// 0x6400 | u is 1024 + u, and subtracting 1152 (packed) leaves b.
__device__ __forceinline__ u32x2 i8x4_to_f16(unsigned w) {
    const unsigned x = w ^ 0x80808080u;
    const unsigned a = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);  // bytes u0, 0x64, u1, 0x64
    const unsigned b = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);  // bytes u2, 0x64, u3, 0x64
    const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    return u32x2{__builtin_bit_cast(unsigned, __builtin_bit_cast(f16x2, a) - bias),
                 __builtin_bit_cast(unsigned, __builtin_bit_cast(f16x2, b) - bias)};
}

// The 16-value V run lane `lane` widens in step i of a Q8_0 tile: (row, kv
// head, run in the head, swap).  The lane reads the run's words 2 s, 2 s + 1
// first (they go to the run's 16-byte V-tile chunk s), then the other two.
// At 2 kv heads (raw rows of 34 words) each 32-lane half takes rows {e, e + 1,
// e + 8, e + 9}, 8 lanes per row, and swaps the second kv head's runs: the
// raw words of each read then fall in 32 distinct banks, and each 8 lanes'
// 16-byte V-tile writes in 8 distinct bank groups (the plain order, 8 lanes
// per row for rows 0..7 and 8..15, conflicts 2-way on both).
template <int KV>
__device__ __forceinline__ int4 q8_vrun(int i, int lane) {
    if constexpr (KV == 2) {
        const int hg = 2 * i + lane / 32, gi = (lane % 32) / 8, h = (lane / 4) % 2;
        return int4{2 * hg + (gi & 1) + 8 * (gi >> 1), h, lane % 4, h};
    } else {
        const int q = 64 * i + lane;
        return int4{q / (4 * KV), (q / 4) % KV, q % 4, 0};
    }
}

// Element type -> MFMA operand type, tile, and cache row bytes.
template <typename T, int KV>
struct MTraits {
    using Ops = MMath<T>;
    using QOps = MMath<T>;
    using Tile = MTile<T, KV>;
    static constexpr int kCacheRowBytes = Tile::ROWB;
};
template <int KV>
struct MTraits<q8_0_t, KV> {
    using Ops = MMath<__bf16>;
    using QOps = MMath<_Float16>;
    using Tile = MTileQ8<KV>;
    static constexpr int kCacheRowBytes = Tile::ROWB;
};

template <typename T, int KV>
__device__ __forceinline__ void mtile_load_any(typename MTraits<T, KV>::Tile& t, const char* kbase,
                                               const char* vbase, int valid, int lane) {
    if constexpr (__is_same(T, q8_0_t))
        mtile_load_q8<KV>(t, kbase, vbase, lane);  // full tiles only (the tail goes through mtile_tail_q8)
    else
        mtile_load<T, KV>(t, kbase, vbase, valid, lane);
}

// One MFMA decode segment: rows r0 .. r0 + n_rows - 1 of sequence seq (base:
// its first cache row in the contiguous modes), merged over the waves and
// written to out_heads (ws_split null) or as this split's partial.  split and
// n_act matter in the layer modes only (the last split writes the new row).
// Every thread of the workgroup calls it.
template <typename T, int G, int KV, int MODE>
__device__ __forceinline__ void mdecode_segment(const DecodeArgs& a, int seq, int split, int n_act, int pos,
                                                size_t base, int r0, int n_rows, float* __restrict__ out_heads,
                                                float* __restrict__ ws_split) {
    constexpr bool Q8 = __is_same(T, q8_0_t);
    using Tile = typename MTraits<T, KV>::Tile;
    using M = typename MTraits<T, KV>::Ops;
    // q . k operand type: the cache's 16-bit type; Q8_0 keys are widened to fp16
    // (exact, i8x4_to_f16), its p . v stays on bf16.
    using MQ = typename MTraits<T, KV>::QOps;
    constexpr int ROWC = MTraits<T, KV>::kCacheRowBytes;  // cache bytes per row
    constexpr int ROWB = KV * kHeadDim * 2;                // bytes per row of the 16-bit LDS V tile
    constexpr int CPR = ROWB / 16, NKB = 2 * KV, NMB = 4 * KV;
    constexpr int NH = KV * G;
    constexpr int NW = mdecode_waves<T>(), D = kMDepth;
    constexpr bool PAGED = is_paged(MODE);
    constexpr bool LAYER = is_layer(MODE);
    static_assert(NH <= 16, "query heads are the 16 MFMA columns");
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, g = lane >> 4;
    const float2* cs_row = LAYER ? a.rope_cs + (size_t)pos * (kHeadDim / 2) : nullptr;

    // Q^T operands: column col, dims 32 (b % 2) + 8 g + 0..7 of kv head b / 2,
    // zero unless head col belongs to that kv head.  16-bit parts, each rounded
    // to nearest from the exact remainder of the previous ones: bf16 three (hi +
    // mid + lo, 24 bits: fp32 exactly), fp16 two (22 bits: |q - hi - lo| <=
    // 2^-22 |q|, below the rounding of fp32 sums of 64 products).  fp16: the
    // column is first scaled by 2^qe (exact), its largest element into
    // [2^14, 2^15): an element's error is then at most max(2^-22 |q|, 2^-25),
    // the second (fp16 subnormal lo parts) below 2^-39 of the largest.
    float qx[NKB][8];
#pragma unroll
    for (int b = 0; b < NKB; ++b) {
        const bool mine = col < NH && col / G == b / 2;
        const float* qp = a.q + ((size_t)seq * NH + min(col, NH - 1)) * kHeadDim + 32 * (b % 2) + 8 * g;
        const float4 x0 = *reinterpret_cast<const float4*>(qp);
        const float4 x1 = *reinterpret_cast<const float4*>(qp + 4);
        float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        if (LAYER) {  // RoPE of pairs (16 (b % 2) + 4 g + t)
            const float4 c0 = *reinterpret_cast<const float4*>(cs_row + 16 * (b % 2) + 4 * g);
            const float4 c1 = *reinterpret_cast<const float4*>(cs_row + 16 * (b % 2) + 4 * g + 2);
            rotate_pair(x[0], x[1], c0.x, c0.y);
            rotate_pair(x[2], x[3], c0.z, c0.w);
            rotate_pair(x[4], x[5], c1.x, c1.y);
            rotate_pair(x[6], x[7], c1.z, c1.w);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) qx[b][t] = mine ? x[t] * a.qscale : 0.f;
    }
    float s_unscale = 1.0f;  // S^T column scale to undo (fp16)
    if (MQ::kScaleQ) {
        float mx = 0.f;
#pragma unroll
        for (int b = 0; b < NKB; ++b)
#pragma unroll
            for (int t = 0; t < 8; ++t) mx = fmaxf(mx, fabsf(qx[b][t]));
        mx = max4_rows(mx);
        int qe = 0;
        if (mx > 0.f) qe = 14 - (int)((__float_as_uint(mx) >> 23) & 0xFF) + 127;  // mx * 2^qe in [2^14, 2^15)
        qe = max(min(qe, 126), -126);
#pragma unroll
        for (int b = 0; b < NKB; ++b)
#pragma unroll
            for (int t = 0; t < 8; ++t) qx[b][t] = __builtin_ldexpf(qx[b][t], qe);
        s_unscale = __builtin_ldexpf(1.0f, -qe);
    }
    constexpr int QP = MQ::kQParts;
    typename MQ::v8 qpart[QP][NKB];
#pragma unroll
    for (int b = 0; b < NKB; ++b) {
        u32x4 w[QP];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float e0 = qx[b][2 * t], e1 = qx[b][2 * t + 1];
#pragma unroll
            for (int part = 0; part < QP; ++part) {
                w[part][t] = MQ::pack2(e0, e1);
                e0 -= MQ::lo(w[part][t]);  // exact
                e1 -= MQ::hi(w[part][t]);
            }
        }
#pragma unroll
        for (int part = 0; part < QP; ++part) qpart[part][b] = __builtin_bit_cast(typename MQ::v8, w[part]);
    }

    // LDS: during the tile loop each wave owns a V tile (16-bit, swizzled) and,
    // for Q8_0, a second V tile (the tile loop is pipelined: one tile's p . v
    // reads one while the next tile is widened into the other) and the raw K
    // and V tiles; after it the same bytes hold the per-wave states for the
    // merge.
    constexpr int VT = kMTileRows * ROWB;
    constexpr int RAWT = Q8 ? MTileQ8<KV>::RAW : 0;
    constexpr bool PIPE = Q8 && NW * (2 * VT + 2 * RAWT) <= 160 * 1024;  // 4 kv heads: 200 KB, not pipelined
    static_assert(!PIPE || D % 2 == 0, "pipelined tile loop: tile j's V tile is j % 2, fixed per unrolled step");
    constexpr int NVT = PIPE ? 2 : 1;
    constexpr int WAVE_LDS = NVT * VT + 2 * RAWT;
    constexpr int NP = NW + (LAYER ? 1 : 0);  // partials merged: the waves, plus the new token in layer modes
    constexpr int MERGE_LDS = NP * NH * kHeadDim * 4 + 2 * NP * NH * 4;
    __shared__ __attribute__((aligned(16))) char smem[NW * WAVE_LDS > MERGE_LDS ? NW * WAVE_LDS : MERGE_LDS];
    char* sv = smem + wave * WAVE_LDS;
    constexpr int NWR = Q8 ? 2 * MTileQ8<KV>::NVU : MTile<__bf16, KV>::NV;  // 16-byte LDS writes per lane
    int wr_off[NWR];
    int vrd_off[NWR];  // Q8_0: raw V byte offsets of the words widened into V-tile write i
#pragma unroll
    for (int i = 0; i < NWR; ++i) {
        int r, c;
        if (Q8) {  // write i: chunk (i & 1) ^ swap of run i / 2 (q8_vrun)
            const int4 u = q8_vrun<KV>(i / 2, lane);
            const int half = (i & 1) ^ u.w;
            r = u.x;
            c = 8 * u.y + 2 * u.z + half;
            vrd_off[i] = r * MTileQ8<KV>::ROWB + u.y * kQ8HeadBytes + 16 * u.z + 8 * half;
        } else {
            const int q = 64 * i + lane;
            r = q / CPR;
            c = q % CPR;
        }
        wr_off[i] = r * ROWB + 16 * (c ^ mswz<KV>(r));
    }
    char* rk = sv + NVT * VT;  // Q8_0: raw K tile
    char* rv = rk + RAWT;  // Q8_0: raw V tile
    int x_off = 0;         // Q8_0: this lane's remainder chunk, from rk
    if constexpr (Q8) {
        const int2 rc = q8_rem_chunk<KV>(lane);
        x_off = rc.x * RAWT + 16 * rc.y;
    }
    int rd_off[NMB];
    {
        const int j = col, r = 4 * g + j / 4;
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
            rd_off[mb] = r * ROWB + 16 * ((2 * mb + (j & 3) / 2) ^ mswz<KV>(r)) + 8 * (j & 1);
    }

    f32x4 acc[NMB];
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = kNegInf, l = 0.f;

    const char* kc = reinterpret_cast<const char*>(a.k) + (PAGED ? 0 : base * ROWC);
    const char* vc = reinterpret_cast<const char*>(a.v) + (PAGED ? 0 : base * ROWC);
    const PageMap pm{PAGED ? a.block_table + (size_t)seq * a.max_pages : nullptr, r0, a.n_pages};
    unsigned bad = 0;
    auto tile_off = [&](int t) -> size_t {  // byte offset of tile t's row 0 from kc / vc
        const int row = r0 + t * kMTileRows;
        if (!PAGED) return (size_t)row * ROWC;
        return (size_t)page_of(pm, row, bad) * kPageRows * ROWC;
    };

    // One tile in two stages.  front: V into the V tile `vt`, S^T = K q (rows
    // past `valid` masked); Q8_0: the raw tile is already in LDS when t is
    // null.  back: online softmax and O^T += V^T P^T from `vt`.
    struct Front {
        f32x4 s;
        f16x2 dv[4];  // Q8_0: V scales (blocks 0, 1 of the own kv head) of this lane's keys 4 g + i
    };
    auto front = [&](const Tile* t, int valid, char* vt) -> Front {
        f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
        f16x2 dv[4] = {};
        if constexpr (Q8) {
            constexpr int RB = MTileQ8<KV>::ROWB;
            if (t) {
#pragma unroll
                for (int i = 0; i < MTileQ8<KV>::NF; ++i) {
                    *reinterpret_cast<u32x4*>(rk + 16 * (64 * i + lane)) = t->k[i];
                    *reinterpret_cast<u32x4*>(rv + 16 * (64 * i + lane)) = t->v[i];
                }
                // Lanes past 2 REM hold and store copies of lanes 0 .. 2 REM - 1's
                // chunks (same address, same bytes): no branch in the tile code.
                *reinterpret_cast<u32x4*>(rk + x_off) = t->x;
            }
#pragma unroll
            for (int i = 0; i < MTileQ8<KV>::NVU; ++i) {  // V runs: widen to bf16, into the V tile
                const unsigned* sa = reinterpret_cast<const unsigned*>(rv + vrd_off[2 * i]);
                const unsigned* sb = reinterpret_cast<const unsigned*>(rv + vrd_off[2 * i + 1]);
                const u32x2 a0 = i8x4_to_bf16(sa[0]), a1 = i8x4_to_bf16(sa[1]);
                const u32x2 a2 = i8x4_to_bf16(sb[0]), a3 = i8x4_to_bf16(sb[1]);
                const u32x4 w0 = {a0[0], a0[1], a1[0], a1[1]}, w1 = {a2[0], a2[1], a3[0], a3[1]};
                *reinterpret_cast<u32x4*>(vt + wr_off[2 * i]) = w0;
                *reinterpret_cast<u32x4*>(vt + wr_off[2 * i + 1]) = w1;
            }
            // Scales of this lane's keys 4 g + i in its own column's kv head only:
            // the other kv head's S^T entries of the column are exactly 0 (its
            // query operand is 0 there), and its P' is never read back.
            // Kept as fp16 pairs: each use is one v_fma_mix_f32 (fp16 operand
            // selected from either half, no conversion).
            const int kvc = min(col, NH - 1) / G;
            f16x2 dk[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int o = (4 * g + i) * RB + kvc * kQ8HeadBytes + 64;
                const bool ok = 4 * g + i < valid;  // rows past the tile's end: weight 0, whatever LDS holds
                const unsigned kw = *reinterpret_cast<const unsigned*>(rk + o);
                const unsigned vw = ok ? *reinterpret_cast<const unsigned*>(rv + o) : 0u;
                dk[i] = __builtin_bit_cast(f16x2, kw);
                dv[i] = __builtin_bit_cast(f16x2, vw);
            }
            // S^T of each 32-dim block parity, both kv heads into one accumulator
            // (the block-diagonal query keeps them apart): K widened to fp16
            // exactly, fp16 MFMAs against the fp16 query parts.
            f32x4 sb[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int b = 0; b < NKB; ++b) {
                const unsigned* src =
                    reinterpret_cast<const unsigned*>(rk + col * RB + (b / 2) * kQ8HeadBytes + 32 * (b % 2) + 8 * g);
                const u32x2 k0 = i8x4_to_f16(src[0]), k1 = i8x4_to_f16(src[1]);
                const u32x4 kw = {k0[0], k0[1], k1[0], k1[1]};
                const typename MQ::v8 kop = __builtin_bit_cast(typename MQ::v8, kw);
#pragma unroll
                for (int part = QP - 1; part >= 0; --part) sb[b % 2] = MQ::mfma32(kop, qpart[part][b], sb[b % 2]);
            }
            // + 0.0f keeps the product a fused multiply-add (one v_fma_mix_f32
            // with the fp16 operand) rather than a conversion and a multiply.
#pragma unroll
            for (int i = 0; i < 4; ++i)
                s[i] = __builtin_fmaf((float)dk[i][0], sb[0][i], __builtin_fmaf((float)dk[i][1], sb[1][i], 0.0f));
        } else {
#pragma unroll
            for (int i = 0; i < NWR; ++i) *reinterpret_cast<u32x4*>(vt + wr_off[i]) = t->v[i];
#pragma unroll
            for (int b = 0; b < NKB; ++b)
#pragma unroll
                for (int part = QP - 1; part >= 0; --part)  // smallest part first
                    s = M::mfma32(t->k[b], qpart[part][b], s);
        }
        if (valid < kMTileRows) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (4 * g + i >= valid) s[i] = kNegInf;
        }
        return Front{s, {dv[0], dv[1], dv[2], dv[3]}};
    };
    auto back = [&](const Front& f, char* vt) {
        const f32x4 s = f.s;
        // fp16 queries: s holds S^T times 2^qe; the power of two comes off
        // the tile max and inside the exp2 argument (exact either way).
        // Every lane tests its own 4 keys: the column's max exceeds m + kTau
        // exactly when one of its 4 lanes' does, and only then (rare after
        // the first tile) is the column max reduced over the lanes.
        float tm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        if (MQ::kScaleQ) tm *= s_unscale;
        if (__any(tm - m > kTau)) {  // raise the running max
            tm = max4_rows(tm);
            const float mn = fmaxf(m, tm);
            const float alpha = (m == kNegInf) ? 0.f : fast_exp2(m - mn);
            l *= alpha;
#pragma unroll
            for (int mb = 0; mb < NMB; ++mb) acc[mb] *= alpha;
            m = mn;
        }
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            p[i] = fast_exp2(MQ::kScaleQ ? __builtin_fmaf(s[i], s_unscale, -m) : s[i] - m);  // 0 for masked keys
            l += p[i];
        }
        // P^T (times kPScale; Q8_0: times the key's V scale of the block) as
        // 16-bit hi + lo, both in one K = 32 operand: k-slots 8 g .. 8 g + 3
        // hold this lane's 4 keys' hi parts, 8 g + 4 .. 8 g + 7 their lo parts,
        // and the V operand repeats the 4 keys' values in both halves (the
        // order of a contraction's k-slots is free): one 16x16x32 MFMA per
        // 16-dim block in place of two 16x16x16 ones.
        constexpr int NP = Q8 ? 2 : 1;  // Q8_0: one P' per 32-dim block of the column's own kv head
        typename M::v8 pv[NP];
#pragma unroll
        for (int b = 0; b < NP; ++b) {
            u32x2 ph, pl;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                float p0 = p[2 * i] * M::kPScale, p1 = p[2 * i + 1] * M::kPScale;
                if constexpr (Q8) {
                    p0 = __builtin_fmaf((float)f.dv[2 * i][b], p0, 0.0f);
                    p1 = __builtin_fmaf((float)f.dv[2 * i + 1][b], p1, 0.0f);
                }
                ph[i] = M::pack2(p0, p1);
                pl[i] = M::pack2(p0 - M::lo(ph[i]), p1 - M::hi(ph[i]));
            }
            pv[b] = M::cat(__builtin_bit_cast(typename M::v4, ph), __builtin_bit_cast(typename M::v4, pl));
        }
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) {
            const typename M::v4 va = M::read_tr(vt + rd_off[mb]);
            const int b = Q8 ? (mb & 3) >> 1 : 0;  // Q8_0: 32-dim block of dims 16 mb .. 16 mb + 15 in its kv head
            acc[mb] = M::mfma32(M::cat(va, va), pv[b], acc[mb]);
        }
    };
    auto compute = [&](const Tile* t, int valid) { back(front(t, valid, sv), sv); };

    const int full = n_rows / kMTileRows;
    const int nk = (full - wave + NW - 1) / NW;  // this wave's full tiles: wave + NW * k
    if (nk > 0) {
        Tile buf[D];
        auto load = [&](int d, int k) {
            const size_t off = tile_off(wave + NW * k);
            mtile_load_any<T, KV>(buf[d], kc + off, vc + off, kMTileRows, lane);
        };
#pragma unroll
        for (int d = 0; d < D; ++d) {
            load(d, min(d, nk - 1));
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (PIPE) {
            // Two-stage pipeline: the front of tile j + 1 is issued before
            // the back of tile j, so the widening, LDS round trips and q . k
            // MFMAs of one tile overlap the softmax and p . v of the other
            // (each alone is a chain of dependent steps that two waves per
            // SIMD do not hide).  Tile j's V tile is j % 2.  Invariant at the
            // loop head: front(k0) done (st), buf[(k0 + 1 + i) % D] holds tile
            // k0 + 1 + i for i < D; loads are unconditional here as in the
            // plain loop below (the first refill is clamped to the last tile).
            Front st = front(&buf[0], kMTileRows, sv);
            load(0, min(D, nk - 1));
            int k0 = 0;
            for (; k0 + 2 * D < nk; k0 += D) {
#pragma unroll
                for (int d = 0; d < D; ++d) {
                    const int n = (d + 1) % D;
                    const Front nx = front(&buf[n], kMTileRows, sv + ((d + 1) & 1) * VT);
                    load(n, k0 + d + 1 + D);
                    back(st, sv + (d & 1) * VT);
                    st = nx;
                }
            }
            // Drain: tiles k0 .. nk - 1 (at most 2 D), front(k0) done.
#pragma unroll
            for (int i = 0; i < 2 * D; ++i) {
                if (k0 + i < nk) {
                    const int n = (i + 1) % D;
                    Front nx = st;
                    if (k0 + i + 1 < nk) {
                        nx = front(&buf[n], kMTileRows, sv + ((i + 1) & 1) * VT);
                        if (k0 + i + 1 + D < nk) load(n, k0 + i + 1 + D);
                    }
                    back(st, sv + (i & 1) * VT);
                    st = nx;
                }
            }
        } else {
            // Steady state: every prefetch is one of the wave's tiles, so every
            // iteration issues the same loads and a tile's compute waits only for
            // that tile's loads (a conditional prefetch makes the compiler wait
            // for all loads in flight, the D - 1 newer tiles included).  No tile
            // is fetched twice (a prefetch clamped to the last tile re-read it).
            int k0 = 0;
            for (; k0 + 2 * D <= nk; k0 += D) {
#pragma unroll
                for (int d = 0; d < D; ++d) {
                    compute(&buf[d], kMTileRows);
                    load(d, k0 + d + D);
                }
            }
            // Drain: the last nk - k0 < 2 D tiles.
#pragma unroll
            for (int d = 0; d < D; ++d) {
                if (k0 + d < nk) compute(&buf[d], kMTileRows);
                if (k0 + d + D < nk) load(d, k0 + d + D);
            }
#pragma unroll
            for (int d = 0; d < D; ++d)
                if (k0 + D + d < nk) compute(&buf[d], kMTileRows);
        }
    }
    const int tail = n_rows - full * kMTileRows;
    if (tail > 0 && (full % NW) == wave) {
        const size_t off = tile_off(full);
        if constexpr (Q8) {
            mtile_tail_q8<KV>(kc + off, vc + off, tail, rk, rv, lane);
            compute(nullptr, tail);
        } else {
            Tile t;
            mtile_load_any<T, KV>(t, kc + off, vc + off, tail, lane);
            compute(&t, tail);
        }
    }
    if (PAGED && bad && lane == 0) atomicOr(a.err, 4);

    // Wave states -> LDS -> merge.  Column col's row sum is spread over the 4
    // lane groups; its output dims 16 mm + 4 g + i live in the M-blocks of its
    // own kv head.
    l = sum4_rows(l);
    if (M::kPScale != 1.0f) {  // O^T accumulated P * kPScale (a power of two)
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) acc[mb] *= 1.0f / M::kPScale;
    }
    __syncthreads();  // every wave is done with its tiles before the merge area reuses them
    auto s_acc = reinterpret_cast<float (*)[NH][kHeadDim]>(smem);
    auto s_m = reinterpret_cast<float (*)[NH]>(smem + NP * NH * kHeadDim * 4);
    auto s_l = reinterpret_cast<float (*)[NH]>(smem + NP * NH * kHeadDim * 4 + NP * NH * 4);
    if (LAYER && wave == 0) {
        // The new token (row pos), as one more partial.  Lanes take the VALU
        // kernels' layout (8 lanes per kv head, dims {4c..4c+3, 32+4c..}): RoPE
        // its k, round / quantize k and v_new to the cache type, write them to
        // the cache row (tmac_gguf.cpp:1090-1091; the last split only) and score
        // them against the rotated, pre-scaled query of each head of the group.
        const int c = lane & 7, kvh = lane >> 3;
        const bool mine = lane < 8 * KV;
        const bool last = split == n_act - 1;
        float kf[8], vf[8];
        if (mine) {
            const int colf = kvh * kHeadDim + 4 * c;
            const size_t in = (MODE == kPagedLayer ? (size_t)seq * KV * kHeadDim : 0) + colf;
            load8(kf, a.k_new + in);
            load8(vf, a.v_new + in);
            rope8(kf, cs_row, c);
            size_t row = (size_t)pos;
            if (PAGED) row = (size_t)page_of(pm, pos, bad) * kPageRows + (pos & (kPageRows - 1));
            const int lane_col = kvh * CacheFmt<T>::kHeadBytes + 4 * c * CacheFmt<T>::kDimBytes;
            put_row<T>(kf, reinterpret_cast<char*>(a.k_out) + row * ROWC + lane_col, c, last);
            put_row<T>(vf, reinterpret_cast<char*>(a.v_out) + row * ROWC + lane_col, c, last);
#pragma unroll
            for (int gq = 0; gq < G; ++gq) {
                const int h = kvh * G + gq;
                float qf[8];
                load8(qf, a.q + ((size_t)seq * NH + h) * kHeadDim + 4 * c);
                rope8(qf, cs_row, c);
                float d = 0.f;
#pragma unroll
                for (int t = 0; t < 8; ++t) d = fmaf(qf[t] * a.qscale, kf[t], d);
                d = slot_sum(d);
                const bool take = last;  // other splits contribute nothing for the new token
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    s_acc[NW][h][4 * c + t] = take ? vf[t] : 0.f;
                    s_acc[NW][h][32 + 4 * c + t] = take ? vf[4 + t] : 0.f;
                }
                if (c == 0) {
                    s_m[NW][h] = take ? d : kNegInf;
                    s_l[NW][h] = take ? 1.f : 0.f;
                }
            }
        }
        if (PAGED && bad && lane == 0) atomicOr(a.err, 4);
    }
    if (col < NH) {
        const int kv = col / G;
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) {
#pragma unroll
            for (int mb = 0; mb < NMB; ++mb) {
                if (mb == 4 * kv + mm) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) s_acc[wave][col][16 * mm + 4 * g + i] = acc[mb][i];
                }
            }
        }
        if (g == 0) {
            s_m[wave][col] = m;
            s_l[wave][col] = l;
        }
    }
    __syncthreads();
    merge_waves<NH, NP, NW * 64>(s_acc, s_m, s_l, ws_split == nullptr, out_heads, ws_split);
}

// MFMA decode for one (split, sequence) workgroup (flat unit grid in the
// ragged and paged modes).
template <typename T, int G, int KV, int MODE>
__device__ __forceinline__ void mdecode_body(const DecodeArgs& a) {
    constexpr int NH = KV * G;
    constexpr int NW = mdecode_waves<T>();
    constexpr bool PAGED = is_paged(MODE);
    constexpr bool LAYER = is_layer(MODE);
    int split = blockIdx.x, seq = blockIdx.y;
    int n_pos, pos;
    size_t base;
    bool geo_ok;
    if (MODE == kRagged || PAGED) {
        const bool by_pos = MODE == kPagedLayer;
        int raw;
        int64_t off;
        if (!ragged_unit(by_pos ? a.positions : a.lengths, MODE == kRagged ? a.offsets : nullptr, by_pos ? 1 : 0,
                         a.n_seq, a.split_len, a.n_splits, blockIdx.x, seq, split, raw, off))
            return;
        geo_ok = unit_geometry<MODE>(a, raw, off, n_pos, pos, base);
    } else {
        geo_ok = seq_geometry<MODE>(a, seq, n_pos, pos, base);
    }
    if (!geo_ok) {
        if (split == 0 && threadIdx.x == 0) atomicOr(a.err, 1);
        return;
    }
    n_pos = __builtin_amdgcn_readfirstlane(n_pos);
    pos = __builtin_amdgcn_readfirstlane(pos);
    float* out_heads = a.out + (size_t)seq * NH * kHeadDim;
    if (n_pos <= 0) {
        if (split == 0)
            for (int i = threadIdx.x; i < NH * kHeadDim; i += NW * 64) out_heads[i] = 0.f;
        return;
    }
    const int n_act = (n_pos + a.split_len - 1) / a.split_len;
    if (n_act > a.n_splits) {
        if (split == 0) {
            for (int i = threadIdx.x; i < NH * kHeadDim; i += NW * 64) out_heads[i] = __builtin_nanf("");
            if (threadIdx.x == 0) atomicOr(a.err, 2);
        }
        return;
    }
    if (split >= n_act) return;
    const int r0 = split * a.split_len;
    const int mem_rows = LAYER ? pos : n_pos;  // layer modes: row `pos` is the new token, attended from registers
    const int n_rows = max(min(r0 + a.split_len, mem_rows) - r0, 0);
    const bool direct = (n_act == 1);
    float* ws_split = direct ? nullptr : a.ws + ((size_t)seq * a.n_splits + split) * NH * kPartialStride;
    mdecode_segment<T, G, KV, MODE>(a, seq, split, n_act, pos, base, r0, n_rows, out_heads, ws_split);
}

// Stream-K decode on the MFMA kernel (bf16 / fp16 / Q8_0 caches, ragged or
// paged): one mdecode_segment per sequence overlapping this workgroup's range
// of the row space.
template <typename T, int G, int KV, bool PAGED>
__device__ __forceinline__ void mdecode_sk_body(const DecodeArgs& a) {
    constexpr int NH = KV * G;
    int64_t S, lo, hi, P;
    int last_u, s, len = 0;
    if (!sk_locate<mdecode_waves<T>() * 64, false>(a, S, lo, hi, last_u, s, P)) return;
    for (bool first = true; sk_seek<false>(a, lo, hi, s, P, len); ++s, first = false) {
        if (!first) __syncthreads();  // the previous segment's merge reads the LDS this one's tiles reuse
        const int64_t r0 = max(lo - P, (int64_t)0), r1 = min(hi - P, (int64_t)len);
        const bool direct = sk_record(a, s, P, len, S, last_u);
        float* ws_slot = direct ? nullptr : a.ws + ((size_t)blockIdx.x + s) * NH * kPartialStride;
        mdecode_segment<T, G, KV, PAGED ? kPaged : kRagged>(a, s, 0, 1, 0, PAGED ? 0 : (size_t)a.offsets[s],
                                                            (int)r0, (int)(r1 - r0),
                                                            a.out + (size_t)s * NH * kHeadDim, ws_slot);
        P += sk_rows(len, a.sk_max_len);
    }
}

#define TMAC_MDECODE_KERNELS_T(G, KV, TN, T)                                                          \
    extern "C" __global__ __launch_bounds__(mdecode_waves<T>() * 64) void tmac_mdecode_u_##TN##_g##G##_kv##KV(     \
        DecodeArgs a) {                                                                                \
        mdecode_body<T, G, KV, kUniform>(a);                                                           \
    }                                                                                                  \
    extern "C" __global__ __launch_bounds__(mdecode_waves<T>() * 64) void tmac_mdecode_r_##TN##_g##G##_kv##KV(     \
        DecodeArgs a) {                                                                                \
        mdecode_body<T, G, KV, kRagged>(a);                                                            \
    }                                                                                                  \
    extern "C" __global__ __launch_bounds__(mdecode_waves<T>() * 64) void tmac_mdecode_p_##TN##_g##G##_kv##KV(     \
        DecodeArgs a) {                                                                                \
        mdecode_body<T, G, KV, kPaged>(a);                                                             \
    }                                                                                                  \
    extern "C" __global__ __launch_bounds__(mdecode_waves<T>() * 64) void tmac_mdecode_l_##TN##_g##G##_kv##KV(     \
        DecodeArgs a) {                                                                                \
        mdecode_body<T, G, KV, kLayer>(a);                                                             \
    }                                                                                                  \
    extern "C" __global__ __launch_bounds__(mdecode_waves<T>() * 64) void tmac_mdecode_pl_##TN##_g##G##_kv##KV(    \
        DecodeArgs a) {                                                                                \
        mdecode_body<T, G, KV, kPagedLayer>(a);                                                        \
    }                                                                                                  \
    extern "C" __global__ __launch_bounds__(mdecode_waves<T>() * 64) void tmac_mdecode_sk_##TN##_g##G##_kv##KV(    \
        DecodeArgs a) {                                                                                \
        mdecode_sk_body<T, G, KV, false>(a);                                                           \
    }                                                                                                  \
    extern "C" __global__ __launch_bounds__(mdecode_waves<T>() * 64) void tmac_mdecode_sk_p_##TN##_g##G##_kv##KV(  \
        DecodeArgs a) {                                                                                \
        mdecode_sk_body<T, G, KV, true>(a);                                                            \
    }
#define TMAC_MDECODE_KERNELS(G, KV)               \
    TMAC_MDECODE_KERNELS_T(G, KV, bf16, __bf16)    \
    TMAC_MDECODE_KERNELS_T(G, KV, f16, _Float16)   \
    TMAC_MDECODE_KERNELS_T(G, KV, q8, q8_0_t)

#if TMAC_IN_PART(3)
TMAC_MDECODE_KERNELS(7, 2)
TMAC_MDECODE_KERNELS(1, 1)
TMAC_MDECODE_KERNELS(1, 2)
TMAC_MDECODE_KERNELS(2, 2)
TMAC_MDECODE_KERNELS(4, 2)
TMAC_MDECODE_KERNELS(4, 4)
TMAC_MDECODE_KERNELS(8, 1)
#endif

#if TMAC_IN_PART(3)  // projection, RoPE, copy, conversion and position kernels
// ---------------------------------------------------------------------------
// QKV projection: the producer of q / k_new / v_new (fused_qkv_op,
// metal_backend.hpp:456-489; CPU form tmac_gguf.cpp:1046-1081, dequantisation
// tmac_gguf.cpp:240-250 and 311-327).  y = W x (+ b) for the three weight
// matrices of a layer in one launch, one wave per output row.  Lane u of a row
// takes half of block u / 2: for Q5_0 the elements 8h + i and 16 + 8h + i
// (i < 8; byte 8h + i of qs holds both nibbles), for Q8_0 the elements 16h + i
// (i < 16).  Every block field sits at an even offset, so the weights are read
// as 16-bit words.  The dequantised weight d * q is exact in fp32; the row sum
// is one fused multiply-add per element, then a wave reduction, so it differs
// from the reference's sequential sum only by rounding (wave_sum).

__device__ __forceinline__ unsigned ld16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

extern "C" __global__ __launch_bounds__(kQkvWaves * 64) void tmac_qkv(QkvArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int r = blockIdx.x * kQkvWaves + wave;
    int seg = 0;
    if (r >= a.rows[0]) {
        r -= a.rows[0];
        seg = 1;
        if (r >= a.rows[1]) {
            r -= a.rows[1];
            seg = 2;
            if (r >= a.rows[2]) return;
        }
    }
    const bool q8 = seg == 2 && a.v_is_q8;
    const int nb = a.cols >> 5;
    const int bytes = q8 ? 34 : 22;
    const uint8_t* wrow = a.w[seg] + (size_t)r * nb * bytes;
    float acc = 0.f;
    for (int u = lane; u < 2 * nb; u += 64) {
        const int b = u >> 1, h = u & 1;
        const uint8_t* blk = wrow + (size_t)b * bytes;
        const float d = half_bits_to_float(ld16(blk));
        const float* xb = a.x + 32 * b;
        if (q8) {
            const float4 x0 = *reinterpret_cast<const float4*>(xb + 16 * h);
            const float4 x1 = *reinterpret_cast<const float4*>(xb + 16 * h + 4);
            const float4 x2 = *reinterpret_cast<const float4*>(xb + 16 * h + 8);
            const float4 x3 = *reinterpret_cast<const float4*>(xb + 16 * h + 12);
            const float xv[16] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w,
                                  x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const unsigned pr = ld16(blk + 2 + 16 * h + 2 * i);
                acc = __builtin_fmaf((float)(int8_t)(pr & 0xFF) * d, xv[2 * i], acc);
                acc = __builtin_fmaf((float)(int8_t)(pr >> 8) * d, xv[2 * i + 1], acc);
            }
        } else {
            const unsigned qh = ld16(blk + 2) | (ld16(blk + 4) << 16);
            const float4 l0 = *reinterpret_cast<const float4*>(xb + 8 * h);
            const float4 l1 = *reinterpret_cast<const float4*>(xb + 8 * h + 4);
            const float4 h0 = *reinterpret_cast<const float4*>(xb + 16 + 8 * h);
            const float4 h1 = *reinterpret_cast<const float4*>(xb + 16 + 8 * h + 4);
            const float xl[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
            const float xh[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const unsigned pr = ld16(blk + 6 + 8 * h + 2 * i);
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int j = 8 * h + 2 * i + t;  // element j and j + 16
                    const unsigned byte = (pr >> (8 * t)) & 0xFF;
                    const int qlo = (int)((byte & 0xF) | (((qh >> j) & 1) << 4)) - 16;
                    const int qhi = (int)((byte >> 4) | (((qh >> (j + 16)) & 1) << 4)) - 16;
                    acc = __builtin_fmaf(d * (float)qlo, xl[2 * i + t], acc);
                    acc = __builtin_fmaf(d * (float)qhi, xh[2 * i + t], acc);
                }
            }
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) {
        const float* bias = a.bias[seg];
        a.y[seg][r] = bias ? acc + bias[r] : acc;
    }
}

// RoPE in place, one lane per (head, pair): tmac_gguf.cpp:992-1003 for one
// tensor, i.e. what rope_op (metal_backend.hpp:381) dispatches.
extern "C" __global__ __launch_bounds__(256) void tmac_rope(RopeArgs a) {
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    const int pairs = a.head_dim / 2;
    const int per_row = a.n_heads * pairs;
    const int row = gid / per_row, rem = gid - row * per_row;
    if (row >= a.n_rows) return;
    const int pos = (a.pos_dev ? *a.pos_dev : a.pos_host) + row;
    if (pos < 0 || pos >= a.rope_rows) {
        if (rem == 0) atomicOr(a.err, 1);
        return;
    }
    const int head = rem / pairs, pair = rem - head * pairs;
    const float2 t = a.rope_cs[(size_t)pos * pairs + pair];
    float2* p = reinterpret_cast<float2*>(a.x + (size_t)row * a.row_stride + (size_t)head * a.head_dim) + pair;
    float2 x = *p;
    rotate_pair(x.x, x.y, t.x, t.y);
    *p = x;
}

// dst[i] = src[i]: the cache-row write of elem_op(2, ...); dst[i] += src[i]:
// the bias / residual add of elem_op(0, ...) (kernel_elem ops 2 and 0).
extern "C" __global__ __launch_bounds__(256) void tmac_copy(CopyArgs a) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < a.n) a.dst[i] = a.add ? a.dst[i] + a.src[i] : a.src[i];
}

// K-quant GEMV (matmul_q4_k / matmul_q6_k, metal_backend.hpp:340-350;
// dequantisation tmac_gguf.cpp:330-397): one wave per output row, lane l takes
// elements 4l .. 4l+3 of each 256-weight super-block, which share one sub-block
// scale (and, for Q4_K, one min).  Super-blocks start at even offsets, so their
// bytes are read as 16-bit words.  Each dequantised weight is the reference's
// expression (Q6_K: d * scale * q, exact; Q4_K: d * sc * q - dmin * m, exact
// products and one rounding); the row sum is one FMA per element and a wave
// reduction.
extern "C" __global__ __launch_bounds__(kQkvWaves * 64) void tmac_matmul_kq(KqArgs a) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * kQkvWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (r >= a.rows) return;
    const int nsb = a.cols >> 8;
    const bool q6 = a.type == 14;
    const int bytes = q6 ? 210 : 144;
    const uint8_t* wrow = a.w + (size_t)r * nsb * bytes;
    float acc = 0.f;
    for (int sb = 0; sb < nsb; ++sb) {
        const uint8_t* blk = wrow + (size_t)sb * bytes;
        const float4 xv = *reinterpret_cast<const float4*>(a.x + 256 * sb + 4 * lane);
        const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
        float w[4];
        if (q6) {
            const int half = lane >> 5, sub = (lane >> 3) & 3, l0 = 4 * (lane & 7);
            const float d = half_bits_to_float(ld16(blk + 208));
            const float dsc = d * (float)(int8_t)blk[192 + half * 8 + (l0 >> 4) + 2 * sub];
            const uint8_t* ql = blk + half * 64 + l0 + ((sub & 1) ? 32 : 0);
            const uint8_t* qh = blk + 128 + half * 32 + l0;
            const unsigned qlw = ld16(ql) | (ld16(ql + 2) << 16);
            const unsigned qhw = ld16(qh) | (ld16(qh + 2) << 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const unsigned lb = (qlw >> (8 * i)) & 0xFF;
                const unsigned lo = sub < 2 ? (lb & 0xF) : (lb >> 4);
                const unsigned hi = ((qhw >> (8 * i)) >> (2 * sub)) & 0x3;
                w[i] = dsc * (float)((int)((hi << 4) | lo) - 32);
            }
        } else {
            const int sbk = lane >> 3, q_pos = 4 * (lane & 7);
            const float d = half_bits_to_float(ld16(blk));
            const float dmin = half_bits_to_float(ld16(blk + 2));
            const uint8_t* sc6 = blk + 4;
            unsigned sc, m;
            if (sbk < 4) {
                sc = sc6[sbk] & 63;
                m = sc6[sbk + 4] & 63;
            } else {
                sc = (sc6[sbk + 4] & 0xF) | ((sc6[sbk - 4] >> 6) << 4);
                m = (sc6[sbk + 4] >> 4) | ((sc6[sbk] >> 6) << 4);
            }
            const uint8_t* qs = blk + 16 + (sbk >> 1) * 32 + q_pos;
            const unsigned qw = ld16(qs) | (ld16(qs + 2) << 16);
            const float dsc = d * (float)sc, dm = dmin * (float)m;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const unsigned b = (qw >> (8 * i)) & 0xFF;
                const unsigned q4 = (sbk & 1) ? (b >> 4) : (b & 0xF);
                w[i] = dsc * (float)q4 - dm;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = __builtin_fmaf(w[i], xs[i], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) a.y[r] = a.bias ? acc + a.bias[r] : acc;
}

// Fills a 16-bit cache from fp32 values, rounding to nearest even.
extern "C" __global__ __launch_bounds__(256) void tmac_cvt16(CvtArgs a) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.n) return;
    if (a.dtype == 1)
        reinterpret_cast<__bf16*>(a.dst)[i] = (__bf16)a.src[i];
    else
        reinterpret_cast<_Float16*>(a.dst)[i] = (_Float16)a.src[i];
}

// Fills a Q8_0 cache from fp32 values: n / 64 head rows, each quantized as
// the layer step quantizes a new row (put_row<q8_0_t>), one 8-lane slot per
// head row.
extern "C" __global__ __launch_bounds__(256) void tmac_cvt_q8(CvtArgs a) {
    const int c = threadIdx.x & 7;
    const int64_t hr = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    const bool ok = hr < a.n / kHeadDim;  // the same for the 8 lanes of a slot
    float x[8];
    if (ok) {
        load8(x, a.src + hr * kHeadDim + 4 * c);
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) x[t] = 0.f;
    }
    put_row<q8_0_t>(x, reinterpret_cast<char*>(a.dst) + hr * kQ8HeadBytes + 4 * c, c, ok);
}

// Device-side position for graph replays: *pos = value, or *pos += value.
// Sets or advances a device-side position; with a row cache (a.slots), also
// writes the RoPE row of the new position into its slot (position % 2),
// tagged with (position, table), for the layer steps that follow.
extern "C" __global__ __launch_bounds__(64) void tmac_pos_update(PosArgs a) {
    __shared__ int s_pos;
    if (threadIdx.x == 0) {
        const int p = a.add ? *a.pos + a.value : a.value;
        *a.pos = p;
        s_pos = p;
    }
    if (!a.slots) return;
    __syncthreads();
    const int p = s_pos;
    if (p < 0 || p >= a.rope_rows) return;
    const int sl = p & 1;
    if (threadIdx.x < 16)
        *reinterpret_cast<float4*>(a.slots + 32 * sl + 2 * threadIdx.x) =
            *reinterpret_cast<const float4*>(a.rope_cs + (size_t)p * (kHeadDim / 2) + 2 * threadIdx.x);
    if (threadIdx.x == 0) {
        const uint64_t tab = reinterpret_cast<uint64_t>(a.rope_cs);
        int* tag = reinterpret_cast<int*>(a.slots + 64) + 4 * sl;
        tag[0] = p;
        tag[1] = (int)(uint32_t)tab;
        tag[2] = (int)(uint32_t)(tab >> 32);
    }
}

#endif  // TMAC_IN_PART(3)
