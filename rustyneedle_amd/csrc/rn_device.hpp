// rn_device.hpp — device primitives shared by the gfx950 kernels.
//
// Every float expression is written in the order the CPU restatement uses; the
// library is compiled with -ffp-contract=off, so `a * b + c` rounds twice and
// fmaf is the only fused operation. Division and sqrtf are correctly rounded
// (hipcc's default -fhip-fp32-correctly-rounded-divide-sqrt).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rn {

constexpr int kWave = 64;

// ops.rs:82-90 — clamp, scale by log2(e), round half away from zero, degree-5
// Horner polynomial in the fraction, times 2^whole assembled from its bits.
__device__ __forceinline__ float fast_exp(float value) {
    const float log2e = 1.44269504088896340736f;
    const float ln2 = 0.693147180559945309417f;
    float clamped = value < -87.0f ? -87.0f : (value > 87.0f ? 87.0f : value);
    float scaled = clamped * log2e;
    float whole = __builtin_roundf(scaled);
    float f = scaled - whole;
    float p = 1.0f + f * (ln2 + f * (0.2402265f + f * (0.05550411f + f * (0.009618129f + f * 0.0013333558f))));
    int exponent = (int)whole + 127;
    return p * __uint_as_float((uint32_t)exponent << 23);
}

// ops.rs:73-76
__device__ __forceinline__ float silu(float value) { return value / (1.0f + fast_exp(-value)); }

// ops.rs:112-118 per element: round half to even, clamp to [-128, 127]; NaN -> 0.
__device__ __forceinline__ int quantise_one(float value, float scale) {
    float q = __builtin_rintf(value / scale);
    q = q < -128.0f ? -128.0f : (q > 127.0f ? 127.0f : q);
    if (q != q) return 0;
    return (int)q;
}

// The code of a quotient already divided by the scale: quantise_one's rounding.
__device__ __forceinline__ int code_of_quotient(float y) {
    float q = __builtin_rintf(y);
    q = q < -128.0f ? -128.0f : (q > 127.0f ? 127.0f : q);
    if (q != q) return 0;
    return (int)q;
}

// The quotients value/scale of quantise_one for E values of a lane, without a
// division per element: y = value * (1/scale) is within 1.5 * 2^-23 * |y| of
// the exact quotient and the correctly rounded quotient within 2^-24 of it, so
// unless y lies within |y| * 2^-21 of a half-integer both round to the same
// integer (a tie would put y on the boundary). When any lane of the wave has a
// value that close, the whole wave takes the exact division instead (a
// wave-uniform branch, so the common path carries no division code). The codes
// are bit-identical to quantise_one for every input, NaN and inf included.
template <int E>
__device__ __forceinline__ void quotients(const float* v, float scale, float* y) {
    const float inv = 1.0f / scale;
    bool near = false;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        y[e] = v[e] * inv;
        const float h = floorf(y[e]) + 0.5f;
        near = near || (fabsf(y[e] - h) <= fabsf(y[e]) * 0x1p-21f + 0x1p-30f);
    }
    if (__any(near)) {
#pragma unroll
        for (int e = 0; e < E; ++e) y[e] = v[e] / scale;
    }
}

// ops.rs:103-110
__device__ __forceinline__ float int8_scale_from_peak(float peak) { return peak > 0.0f ? peak / 127.0f : 1.0f; }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        uint64_t other = __shfl_xor(v, o, kWave);
        v = other > v ? other : v;
    }
    return v;
}

// Four int8 x int8 products added to an int32 accumulator (v_dot4_i32_i8).
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

__device__ __forceinline__ int dot16(const int4& w, const int4& x, int c) {
    c = dot4(w.x, x.x, c);
    c = dot4(w.y, x.y, c);
    c = dot4(w.z, x.z, c);
    c = dot4(w.w, x.w, c);
    return c;
}

// Greedy key for generator.rs:257-265: larger float first, then lower index.
// NaN maps to 0 so it never wins; a NaN at index 0 is handled by the caller.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t index) {
    if (v != v) return 0ull;
    if (v == 0.0f) v = 0.0f;  // -0 and +0 compare equal
    uint32_t b = __float_as_uint(v);
    uint32_t ordered = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)ordered << 32) | (uint64_t)(0xffffffffu - index);
}

__device__ __forceinline__ uint32_t argmax_index(uint64_t key) {
    return key == 0ull ? 0u : 0xffffffffu - (uint32_t)(key & 0xffffffffull);
}

}  // namespace rn
