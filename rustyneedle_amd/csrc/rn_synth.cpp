// rn_synth.cpp — seeded synthetic inputs (host memory).
//
// The reference has no random inputs (its bench uses arithmetic token ids,
// crates/bench/src/timing.rs:28-30); the synthetic configurations need seeded
// weights, caches and token ids. Each tensor draws from its own SplitMix64
// stream whose state starts at seed ^ FNV-1a-64(name), so any tensor can be
// regenerated on its own and in any order.
//   codes   : U{-127..127}      from the high 32 bits, (hi * 255) >> 32
//   uniform : lo + (hi-lo) * u  with u = (z >> 40) / 2^24, in double, rounded once
//   normal  : Box-Muller in double with u1 = ((z1 >> 40) + 1) / 2^24, u2 = (z2 >> 40) / 2^24
//   tokens  : (hi * vocab) >> 32
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "../../include/rustyneedle.h"

namespace {

inline uint64_t fnv1a(const char* s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (; *s; ++s) {
        h ^= (uint8_t)*s;
        h *= 0x100000001b3ull;
    }
    return h;
}

struct Stream {
    uint64_t state;
    Stream(uint64_t seed, const char* name) : state(seed ^ fnv1a(name)) {}
    uint64_t next() {
        state += 0x9E3779B97F4A7C15ull;
        uint64_t z = state;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double unit() { return (double)(next() >> 40) * (1.0 / 16777216.0); }
    double normal() {
        const double u1 = ((double)(next() >> 40) + 1.0) * (1.0 / 16777216.0);
        const double u2 = (double)(next() >> 40) * (1.0 / 16777216.0);
        return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925 * u2);
    }
};

// IEEE binary16, round to nearest even.
uint16_t to_half(float value) {
    uint32_t x;
    memcpy(&x, &value, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t mag = x & 0x7fffffffu;
    if (mag > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (mag >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (mag < 0x38800000u) {
        if (mag < 0x33000000u) return (uint16_t)sign;
        const uint32_t mant = (mag & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int)(mag >> 23);
        uint32_t q = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u), halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (((mag >> 23) - 112u) << 10) | ((mag & 0x7fffffu) >> 13);
    const uint32_t rem = mag & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}

}  // namespace

extern "C" {

int rn_synth_codes(uint64_t seed, const char* name, int8_t* out, size_t n) {
    if (!name || (!out && n)) return RN_ERR_ARGUMENT;
    Stream s(seed, name);
    for (size_t i = 0; i < n; ++i) out[i] = (int8_t)((int)(((s.next() >> 32) * 255ull) >> 32) - 127);
    return RN_OK;
}

int rn_synth_uniform(uint64_t seed, const char* name, float lo, float hi, float* out, size_t n) {
    if (!name || (!out && n)) return RN_ERR_ARGUMENT;
    Stream s(seed, name);
    for (size_t i = 0; i < n; ++i) out[i] = (float)((double)lo + ((double)hi - (double)lo) * s.unit());
    return RN_OK;
}

int rn_synth_normal(uint64_t seed, const char* name, float sigma, float* out, size_t n) {
    if (!name || (!out && n)) return RN_ERR_ARGUMENT;
    Stream s(seed, name);
    for (size_t i = 0; i < n; ++i) out[i] = (float)(s.normal() * (double)sigma);
    return RN_OK;
}

int rn_synth_normal_f16(uint64_t seed, const char* name, uint16_t* out, size_t n) {
    if (!name || (!out && n)) return RN_ERR_ARGUMENT;
    Stream s(seed, name);
    for (size_t i = 0; i < n; ++i) out[i] = to_half((float)s.normal());
    return RN_OK;
}

int rn_synth_tokens(uint64_t seed, const char* name, uint32_t vocab, uint32_t* out, size_t n) {
    if (!name || (!out && n) || vocab == 0) return RN_ERR_ARGUMENT;
    Stream s(seed, name);
    for (size_t i = 0; i < n; ++i) out[i] = (uint32_t)(((s.next() >> 32) * (uint64_t)vocab) >> 32);
    return RN_OK;
}

}  // extern "C"
