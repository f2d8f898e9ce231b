// tmac_synth.cpp -- synthetic workload streams for the benchmark and tests.
//
// The benchmark configurations draw their q/k/v values from fixed, seeded
// streams so that a benchmark run and a parity test see the same inputs:
// splitmix64 (Steele, Lea, Flood 2014) expands a 64-bit seed into the state of
// xoshiro256** (Blackman, Vigna 2018); uniforms are the top 53 bits of an
// output scaled by 2^-53; normals come in pairs from the Box-Muller transform
// in double precision (cos first, then sin), each rounded to fp32.
//
// No counterpart in the reference (it reads model weights and prompt tokens);
// this is host code with no GPU use.  Built with -ffp-contract=off and
// -fno-builtin so that the double-precision libm calls and products round
// exactly as written.
#include <cmath>
#include <cstddef>
#include <cstdint>

#include "tmac_attn.h"

namespace {

struct Stream {
    uint64_t s[4];
    bool has_spare = false;
    double spare = 0.0;
};

uint64_t splitmix_next(uint64_t* x) {
    uint64_t z = (*x += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t rotl(uint64_t v, int k) { return (v << k) | (v >> (64 - k)); }

void stream_seed(Stream* st, uint64_t seed) {
    uint64_t x = seed;
    for (auto& w : st->s) w = splitmix_next(&x);
    st->has_spare = false;
}

uint64_t stream_next(Stream* st) {
    uint64_t* s = st->s;
    const uint64_t out = rotl(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return out;
}

double stream_uniform(Stream* st) { return (double)(stream_next(st) >> 11) * 0x1.0p-53; }

float stream_normal(Stream* st) {
    if (st->has_spare) {
        st->has_spare = false;
        return (float)st->spare;
    }
    const double u1 = 1.0 - stream_uniform(st);  // (0, 1]: the logarithm stays finite
    const double u2 = stream_uniform(st);
    const double radius = std::sqrt(-2.0 * std::log(u1));
    const double angle = 6.283185307179586476925286766559 * u2;
    st->spare = radius * std::sin(angle);
    st->has_spare = true;
    return (float)(radius * std::cos(angle));
}

}  // namespace

extern "C" {

int tmac_synth_normal(uint64_t seed, float* out, size_t n) {
    if (!out && n) return TMAC_ERR_NULL_POINTER;
    Stream st;
    stream_seed(&st, seed);
    for (size_t i = 0; i < n; i++) out[i] = stream_normal(&st);
    return TMAC_OK;
}

int tmac_synth_uniform(uint64_t seed, double* out, size_t n) {
    if (!out && n) return TMAC_ERR_NULL_POINTER;
    Stream st;
    stream_seed(&st, seed);
    for (size_t i = 0; i < n; i++) out[i] = stream_uniform(&st);
    return TMAC_OK;
}

}  // extern "C"
