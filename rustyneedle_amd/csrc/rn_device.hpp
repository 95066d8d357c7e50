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

// Native 4-int vector: the i8 MFMA accumulator; arrays of it stay in registers
// where arrays of HIP's int4 struct can be moved to scratch or LDS.
typedef int v4i __attribute__((ext_vector_type(4)));

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

// 2^(i/32) rounded to double, each less i << 47 so that adding k << 47 to the
// entry of k mod 32 gives the bits of 2^(k/32).
static __device__ __constant__ const uint64_t kExp2Table[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

// The C library's expf, which the reference's f32::exp calls (sigmoid,
// ops.rs:68-71; sinkhorn_in_place, ops.rs:198-217; the probe heads' online
// softmax, heads.rs:138-150), as glibc builds it for x86-64 with FMA: the
// method of ARM's optimized-routines expf (Szabolcs Nagy, 2017). With
// z = x * 32/ln2 and k = round(z), exp(x) = 2^(k/32) * 2^(r/32) for r = z - k,
// the second factor a cubic in r; all in double, the reduction and the
// polynomial as fused multiply-adds, one rounding to float at the end. Equal to
// glibc 2.35's expf on every one of the 2^32 inputs.
__device__ __forceinline__ float libm_expf(float x) {
    const uint32_t bits = __float_as_uint(x), magnitude = bits & 0x7fffffffu;
    if (magnitude >= 0x42b00000u) {  // |x| >= 88, infinities, NaN
        if (bits == 0xff800000u) return 0.0f;
        if (magnitude >= 0x7f800000u) return x + x;
        if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_32 = 0x1.71547652b82fep+0 * 32.0, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32768.0, c1 = 0x1.ebfce50fac4f3p-3 / 1024.0,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_32, xd, shift);  // k in the low mantissa bits
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_32, xd, -kd);
    const double s = __longlong_as_double((long long)(kExp2Table[ki % 32] + (ki << 47)));
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return (float)(y * s);
}

// 1.0f / x correctly rounded, for x in [2^-126, 2^126) (positive normal with a
// normal reciprocal): r = v_rcp_f32(x) (within one ulp), then one Newton step
// with fused multiply-adds, r + r (1 - x r). Equal to the IEEE division on
// every float of that range (all 2^31 - 2^25 of them, tests/test_reciprocal.py);
// callers keep x inside it. Three dependent operations against the division's
// nine.
__device__ __forceinline__ float reciprocal_normal(float x) {
    const float r = __builtin_amdgcn_rcpf(x);
    return __builtin_fmaf(__builtin_fmaf(-x, r, 1.0f), r, r);
}

// 1.0f / x for every float: reciprocal_normal inside its range, the IEEE
// division outside it (zero, infinity, NaN, the extremes), on the lanes that
// need it.
__device__ __forceinline__ float reciprocal(float x) {
    if (__builtin_expect(x >= 0x1p-126f && x < 0x1p126f, 1)) return reciprocal_normal(x);
    return 1.0f / x;
}

// ops.rs:68-71 with the C library's expf.
__device__ __forceinline__ float libm_sigmoid(float value) { return reciprocal(1.0f + libm_expf(-value)); }

// The (1/c, log c) pairs of the 16 subintervals of [0x1.66p-1, 0x1.66p0) in
// which the mantissa of x is reduced (rounded to double, as published with the
// method below).
static __device__ __constant__ const double kLogfTable[16][2] = {
    {0x1.661ec79f8f3bep+0, -0x1.57bf7808caadep-2}, {0x1.571ed4aaf883dp+0, -0x1.2bef0a7c06ddbp-2},
    {0x1.49539f0f010bp+0, -0x1.01eae7f513a67p-2},  {0x1.3c995b0b80385p+0, -0x1.b31d8a68224e9p-3},
    {0x1.30d190c8864a5p+0, -0x1.6574f0ac07758p-3}, {0x1.25e227b0b8eap+0, -0x1.1aa2bc79c81p-3},
    {0x1.1bb4a4a1a343fp+0, -0x1.a4e76ce8c0e5ep-4}, {0x1.12358f08ae5bap+0, -0x1.1973c5a611cccp-4},
    {0x1.0953f419900a7p+0, -0x1.252f438e10c1ep-5}, {0x1p+0, 0x0p+0},
    {0x1.e608cfd9a47acp-1, 0x1.aa5aa5df25984p-5},  {0x1.ca4b31f026aap-1, 0x1.c5e53aa362eb4p-4},
    {0x1.b2036576afce6p-1, 0x1.526e57720db08p-3},  {0x1.9c2d163a1aa2dp-1, 0x1.bc2860d22477p-3},
    {0x1.886e6037841edp-1, 0x1.1058bc8a07ee1p-2},  {0x1.767dcf5534862p-1, 0x1.4043057b6ee09p-2}};

// The C library's logf, which the reference's f32::ln calls (the log-mel
// features, frontend.rs:96-99): the method of ARM's optimized-routines logf
// (Szabolcs Nagy, 2017), which glibc builds since 2.28. x = 2^k z with z in
// [0x1.66p-1, 0x1.66p0) and c near the middle of z's subinterval;
// log(x) = k ln2 + log(c) + log1p(r) with r = z/c - 1 = fma(z, 1/c, -1), the
// log1p a cubic in r evaluated in double, one rounding to float at the end.
// Equal to this image's glibc logf on every one of the 2^32 inputs.
__device__ __forceinline__ float libm_logf(float x) {
    uint32_t ix = __float_as_uint(x);
    if (ix == 0x3f800000u) return 0.0f;                      // log(1) = +0 in every rounding mode
    if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {    // subnormal, zero, negative, inf or NaN
        if (ix * 2u == 0u) return -__builtin_inff();
        if (ix == 0x7f800000u) return x;
        if ((ix & 0x80000000u) || ix * 2u >= 0xff000000u) return __builtin_nanf("");
        ix = __float_as_uint(x * 0x1p23f);                   // normalise a subnormal
        ix -= 23u << 23;
    }
    const double ln2 = 0x1.62e42fefa39efp-1;
    const double a0 = -0x1.00ea348b88334p-2, a1 = 0x1.5575b0be00b6ap-2, a2 = -0x1.ffffef20a4123p-2;
    const uint32_t tmp = ix - 0x3f330000u;
    const int i = (int)((tmp >> 19) % 16u);
    const int k = (int32_t)tmp >> 23;
    const uint32_t iz = ix - (tmp & (0x1ffu << 23));
    const double z = (double)__uint_as_float(iz);
    const double r = __builtin_fma(z, kLogfTable[i][0], -1.0);
    const double y0 = kLogfTable[i][1] + (double)k * ln2;
    const double r2 = r * r;
    double y = a1 * r + a2;
    y = a0 * r2 + y;
    y = y * r2 + (y0 + r);
    return (float)y;
}

// The code of a quotient already divided by the scale (ops.rs:112-118 per
// element): round half to even, clamp to [-128, 127], NaN -> 0. Three
// instructions: v_rndne_f32; v_cvt_i32_f32, which saturates out-of-range values
// (infinities included) and converts NaN to 0; v_med3_i32 for the clamp. Equal
// to the select form rint / clamp / NaN test / convert on all 2^32 inputs
// (checked exhaustively on the device).
__device__ __forceinline__ int code_of_quotient(float y) {
    int i;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(i) : "v"(__builtin_rintf(y)));
    return min(max(i, -128), 127);
}

// ops.rs:112-118 per element: the code of value / scale.
__device__ __forceinline__ int quantise_one(float value, float scale) { return code_of_quotient(value / scale); }

// The quotients value/scale of quantise_one for E values of a lane, without a
// division per element: with r = v_rcp_f32(scale), within 1 ulp of 1/scale for
// scales in [2^-100, 2^100], y = value * r is within 1.5 * 2^-23 * |y| of the
// exact quotient and the correctly rounded quotient within 2^-24 of it, so
// unless y lies within |y| * 2^-21 of a half-integer both round to the same
// integer (a tie would put y on the boundary). When any lane of the wave has a
// value that close, or the scale lies outside that range, the whole wave takes
// the exact division instead (a wave-uniform branch, so the common path carries
// no division code). The codes are bit-identical to quantise_one for every
// input, NaN and inf included.
//
// The distance to the half-integer is |fract(y) - 1/2|: exact for y >= 0 and
// |y| >= 1; for y in (-1, 0) fract(y) = fl(y + 1) moves it by at most 2^-25,
// far inside the margin of the bound (|y| 2^-21 against the 1.5 |y| 2^-23 the
// argument needs). Against floor(y) + 1/2 it differs on one input of all 2^32
// (checked on the device), where it takes the exact division.
template <int E>
__device__ __forceinline__ void quotients(const float* v, float scale, float* y) {
    const float inv = __builtin_amdgcn_rcpf(scale);
    bool near = !(scale >= 0x1p-100f && scale <= 0x1p+100f);
#pragma unroll
    for (int e = 0; e < E; ++e) {
        y[e] = v[e] * inv;
        const float d = __builtin_amdgcn_fractf(y[e]) - 0.5f;
        near = near || (fabsf(d) <= __builtin_fmaf(fabsf(y[e]), 0x1p-21f, 0x1p-30f));
    }
    if (__any(near)) {
#pragma unroll
        for (int e = 0; e < E; ++e) y[e] = v[e] / scale;
    }
}

// ops.rs:103-110: peak / 127 (1.0 when the peak is not positive). The quotient
// is formed without a division: q0 = peak * RN(1/127), then one fma correction
// with the exact residual peak - 127 q0; the result equals the correctly
// rounded peak / 127 for every positive finite float (checked exhaustively on
// the CPU over all 2^31 - 2^23 - 1 of them), and an infinite peak stays infinite.
__device__ __forceinline__ float int8_scale_from_peak(float peak) {
    constexpr float kInv127 = 1.0f / 127.0f;
    const float q0 = peak * kInv127;
    const float q = fmaf(fmaf(-q0, 127.0f, peak), kInv127, q0);
    return peak > 0.0f ? (peak == __builtin_inff() ? peak : q) : 1.0f;
}

// The s_waitcnt immediate that waits until at most n (0..63) vector memory
// operations of the wave are outstanding, and for nothing else (gfx9
// encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 at their
// maxima).
constexpr unsigned vmcnt_imm(unsigned n) { return (n & 0xfu) | (((n >> 4) & 3u) << 14) | 0x0f70u; }

// A barrier of the block for its LDS traffic: this wave's LDS operations
// complete, then s_barrier. Unlike __syncthreads it does not wait for the
// wave's global loads and stores, so loads (also into LDS, global_load_lds)
// issued earlier stay in flight across it, and so do stores the block does not
// read back; a kernel reads LDS-bound load data only after an explicit vmcnt
// wait and a barrier. For code whose threads share data through LDS only.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// The same for the lanes of one wave (a one-wave block, or data a wave shares
// with itself): its LDS writes are visible to its later LDS reads.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Cross-lane moves inside rows of 16 lanes (DPP: no LDS round trip). CTRL:
// quad_perm [1,0,3,2] = 0xb1, quad_perm [2,3,0,1] = 0x4e, the quad broadcasts
// 0x00, 0x55, 0xaa, 0xff, row_ror 4 / 8 / 12 = 0x124 / 0x128 / 0x12c,
// row_half_mirror = 0x141, row_mirror = 0x140: every lane has a source lane in
// its row, which must be active. The move carries no old value (a lane whose
// source were disabled would read 0), so the compiler folds it into the
// instruction that consumes it (v_add_f32_dpp and the like: no separate move
// and no wait states between them).
template <int CTRL>
__device__ __forceinline__ int dpp_move(int v) {
    static_assert((CTRL >= 0x00 && CTRL <= 0xff) || CTRL == 0x124 || CTRL == 0x128 || CTRL == 0x12c ||
                      CTRL == 0x140 || CTRL == 0x141,
                  "controls whose every lane has a source in its row");
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true);
}
__device__ __forceinline__ float lane_float(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// The value of lane (this lane ^ M) of a wave, M a power of two up to 32,
// without an LDS round trip: quad_perm for 1 and 2, row rotations by 4 and 12
// (bit 2 picks) and by 8 inside rows of 16, the gfx950 lane swaps for 16
// (v_permlane16_swap: odd rows read the first result, even rows the second)
// and 32 (v_permlane32_swap: the upper half reads the first result, the lower
// the second). Every lane of the wave must be active (a DPP source lane that
// is off yields the lane's own value).
template <int M>
__device__ __forceinline__ int lane_xor_i(int v) {
    if constexpr (M == 1) {
        return dpp_move<0xb1>(v);
    } else if constexpr (M == 2) {
        return dpp_move<0x4e>(v);
    } else if constexpr (M == 4) {
        const int a = dpp_move<0x124>(v), b = dpp_move<0x12c>(v), m = -(((int)threadIdx.x >> 2) & 1);
        return (a & m) | (b & ~m);
    } else if constexpr (M == 8) {
        return dpp_move<0x128>(v);
    } else if constexpr (M == 16) {
        const auto s = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
        const int m = -(((int)threadIdx.x >> 4) & 1);
        return ((int)s[0] & m) | ((int)s[1] & ~m);
    } else {
        static_assert(M == 32, "lane_xor: 1, 2, 4, 8, 16 or 32");
        const auto s = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
        const int m = -(((int)threadIdx.x >> 5) & 1);
        return ((int)s[0] & m) | ((int)s[1] & ~m);
    }
}
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
    return __int_as_float(lane_xor_i<M>(__float_as_int(v)));
}

// Maximum over the 64 lanes of a full wave, the same in every lane. The
// maximum is order-free, so any reduction order gives the same value.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __int_as_float(dpp_move<0xb1>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_move<0x4e>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_move<0x141>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_move<0x140>(__float_as_int(v))));
    return fmaxf(fmaxf(lane_float(v, 0), lane_float(v, 16)), fmaxf(lane_float(v, 32), lane_float(v, 48)));
}

// wave_max for values that are never negative or NaN (the peaks of |x| built
// by fmaxf from 0, which drops NaN): their bit patterns order as the values
// do, so the steps are integer maxima, which the compiler folds with their
// lane moves into one DPP instruction each.
__device__ __forceinline__ float wave_max_nonneg(float v) {
    // (bound_ctrl: a lane without a source would read 0, the identity of the
    // maximum; these lane patterns give every lane a source)
    uint32_t u = __float_as_uint(v);
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0xb1, 0xf, 0xf, true));
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x4e, 0xf, 0xf, true));
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x141, 0xf, 0xf, true));
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x140, 0xf, 0xf, true));
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)u, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)u, 16),
                   c = (uint32_t)__builtin_amdgcn_readlane((int)u, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)u, 48);
    return __uint_as_float(max(max(a, b), max(c, d)));
}

template <int CTRL>
__device__ __forceinline__ uint64_t max_with_dpp_u64(uint64_t v) {
    const uint32_t lo = (uint32_t)dpp_move<CTRL>((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)dpp_move<CTRL>((int)(uint32_t)(v >> 32));
    const uint64_t other = ((uint64_t)hi << 32) | lo;
    return other > v ? other : v;
}
__device__ __forceinline__ uint64_t lane_u64(uint64_t v, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = max_with_dpp_u64<0xb1>(v);
    v = max_with_dpp_u64<0x4e>(v);
    v = max_with_dpp_u64<0x141>(v);
    v = max_with_dpp_u64<0x140>(v);
    const uint64_t a = lane_u64(v, 0), b = lane_u64(v, 16), c = lane_u64(v, 32), d = lane_u64(v, 48);
    const uint64_t ab = b > a ? b : a, cd = d > c ? d : c;
    return cd > ab ? cd : ab;
}

// ops.rs:14-16: the eight lane sums (held by lanes 0..7) added in lane order.
__device__ __forceinline__ float sum_lanes_0_to_7(float s) {
    float total = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) total = total + lane_float(s, q);
    return total;
}

// -0.0 in a register the compiler cannot see into: with a literal -0.0 it
// would turn fma(x, h, -0) back into a conversion and a multiply.
__device__ __forceinline__ float opaque_negative_zero() {
    float z;
    asm("v_mov_b32 %0, 0x80000000" : "=v"(z));
    return z;
}

// x times the f16 in the low (HI false) or high half of `packed`, as one
// v_fma_mix_f32 with a -0.0 addend instead of a conversion and a multiply (the
// compiler selects it from the fma of the widened half, with op_sel for the
// high half, and schedules it as its own instruction, not an opaque asm).
// The f16 operand widens exactly, and fma(x, h, -0) = RN(x h + (-0)) = RN(x h)
// for every operand (a zero product keeps its sign: +0 + -0 = +0, -0 + -0 =
// -0; NaN and infinities pass through), so the result is the product's bits
// whichever instructions compute it.
template <bool HI>
__device__ __forceinline__ float mul_f16(float x, uint32_t packed) {
    const unsigned short bits = HI ? (unsigned short)(packed >> 16) : (unsigned short)(packed & 0xffffu);
    return __builtin_fmaf(x, __half2float(__ushort_as_half(bits)), opaque_negative_zero());
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

__device__ __forceinline__ int dot16(const v4i& w, const int4& x, int c) {
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

// E consecutive floats (E even) with the widest aligned loads.
template <int E>
__device__ __forceinline__ void load_floats(const float* src, float* v) {
    if constexpr (E % 4 == 0) {
#pragma unroll
        for (int e = 0; e < E; e += 4) {
            const float4 t = *reinterpret_cast<const float4*>(src + e);
            v[e] = t.x;
            v[e + 1] = t.y;
            v[e + 2] = t.z;
            v[e + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int e = 0; e < E; e += 2) {
            const float2 t = *reinterpret_cast<const float2*>(src + e);
            v[e] = t.x;
            v[e + 1] = t.y;
        }
    }
}

}  // namespace rn
