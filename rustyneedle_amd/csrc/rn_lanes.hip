// rn_lanes.hip — the multi-lane hyper-connection of Needle 3 (crates/model/src/
// lanes.rs) on gfx950: LaneWeights::route and combine_into around the three
// codebook products of the routing matrices.
//
//   lanes_prologue_kernel: unit_rms of the whole stream (ops.rs:60-66, the
//     eight-lane sum of squares of ops.rs:7-17) and fake_quantise_int8
//     (ops.rs:120-125), one block;
//   the products: rn_codebook.hip on row ranges of phi_pre, phi_post, phi_res;
//   lanes_route_kernel: the gates (sigmoid, ops.rs:68-71), the gated input
//     mix, the post gains, the residual mixing logits and sinkhorn_in_place
//     (ops.rs:198-217), lanes.rs:62-83;
//   lanes_combine_kernel: lanes.rs:86-98.
// sigmoid and sinkhorn use libm_expf, the C library's expf the reference calls.
#include "rn_device.hpp"
#include "rn_internal.hpp"

namespace rn {

constexpr int kLaneThreads = 256;

constexpr int kLaneStage = 8192;  // streams up to this many values are read once into LDS

__global__ __launch_bounds__(256) void lanes_prologue_kernel(const float* stream, int n, float* out) {
    __shared__ float v_s[kLaneStage];
    __shared__ float lanes_s[8];
    __shared__ float peak_s[kLaneThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool staged = n <= kLaneStage;
    if (staged) {
        for (int i = tid; i < n; i += kLaneThreads) v_s[i] = stream[i];
        __syncthreads();
    }
    const float* v = staged ? v_s : stream;
    if (tid < 8) {  // ops.rs:7-17: lane j sums x[8c + j]^2 over c in order
        float s = 0.0f;
        for (int c = 0; c < n / 8; ++c) {
            const float x = v[8 * c + tid];
            s = s + x * x;
        }
        lanes_s[tid] = s;
    }
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) total = total + lanes_s[j];
    total = total + 0.0f;  // the empty tail (n is a multiple of 8)
    const float inverse = reciprocal(sqrtf(total / (float)n + 1e-6f));
    float peak = 0.0f;
    for (int i = tid; i < n; i += kLaneThreads) peak = fmaxf(peak, fabsf(v[i] * inverse));
    peak = wave_max_nonneg(peak);
    if (lane == 0) peak_s[wave] = peak;
    __syncthreads();
    peak = fmaxf(fmaxf(peak_s[0], peak_s[1]), fmaxf(peak_s[2], peak_s[3]));
    const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    for (int i = tid; i < n; i += kLaneThreads) {
        float q = __builtin_rintf((v[i] * inverse) / scale);
        q = q < -128.0f ? -128.0f : (q > 127.0f ? 127.0f : q);
        out[i] = q * scale;
    }
}

// The gates (lanes < L), then the residual mixing logits and their Sinkhorn
// normalisation with one wave lane per entry (L * L <= 64): a row or column
// sum reads the L entries through shuffles in index order, so every lane of a
// row (column) adds the same values in the reference's order.
__global__ __launch_bounds__(256) void lanes_route_kernel(LanesRouteParams p) {
    __shared__ float gate_s[kMaxLanes];
    __shared__ float m_s[kMaxLanes * kMaxLanes];
    const int tid = threadIdx.x, L = p.lanes, own = p.slot % L, n = L * L;
    if (tid < 64) {
        if (tid < L) {
            const int lane = tid;
            const float pre_offset = lane == own ? 8.0f + -4.0f : -4.0f;  // PRE_LANE_BOOST, PRE_LANE_FLOOR
            gate_s[lane] = libm_sigmoid(p.a_pre[p.layer] * p.pre[lane] + p.b_pre[p.layer * L + lane] + pre_offset);
            const float post_offset = lane == own ? 0.0f : -4.0f;  // POST_LANE_FLOOR
            p.post[lane] = 2.0f * libm_sigmoid(p.a_post[p.layer] * p.post[lane] + p.b_post[p.layer * L + lane] +
                                               post_offset);
        }
        if (n <= 64) {
            const int i = tid;
            const bool live = i < n;
            const int r = live ? i / L : 0, c = live ? i % L : 0;
            float m = live ? p.a_res[p.layer] * p.residual[i] + p.b_res[p.layer * n + i] : 0.0f;
            float peak = -INFINITY;  // ops.rs:199-202
            for (int j = 0; j < L; ++j) peak = fmaxf(peak, __shfl(m, r * L + j, 64));
            m = libm_expf(m - peak);
            for (int it = 0; it < 20; ++it) {  // SINKHORN_ITERATIONS; sums fold from -0.0
                float total = -0.0f;
                for (int j = 0; j < L; ++j) total = total + __shfl(m, r * L + j, 64);
                m = m * (1.0f / fmaxf(total, 1.17549435e-38f));
                total = -0.0f;
                for (int j = 0; j < L; ++j) total = total + __shfl(m, j * L + c, 64);
                m = m * (1.0f / fmaxf(total, 1.17549435e-38f));
            }
            if (live) p.residual[i] = m;
        } else if (tid == 0) {  // wide lane counts: one thread over an LDS copy
            float* m = m_s;
            const int base = p.layer * n;
            for (int i = 0; i < n; ++i) m[i] = p.a_res[p.layer] * p.residual[i] + p.b_res[base + i];
            for (int r = 0; r < L; ++r) {
                float peak = -INFINITY;
                for (int c = 0; c < L; ++c) peak = fmaxf(peak, m[r * L + c]);
                for (int c = 0; c < L; ++c) m[r * L + c] = libm_expf(m[r * L + c] - peak);
            }
            for (int it = 0; it < 20; ++it) {
                for (int r = 0; r < L; ++r) {
                    float total = -0.0f;
                    for (int c = 0; c < L; ++c) total = total + m[r * L + c];
                    const float inv = 1.0f / fmaxf(total, 1.17549435e-38f);
                    for (int c = 0; c < L; ++c) m[r * L + c] = m[r * L + c] * inv;
                }
                for (int c = 0; c < L; ++c) {
                    float total = -0.0f;
                    for (int r = 0; r < L; ++r) total = total + m[r * L + c];
                    const float inv = 1.0f / fmaxf(total, 1.17549435e-38f);
                    for (int r = 0; r < L; ++r) m[r * L + c] = m[r * L + c] * inv;
                }
            }
            for (int i = 0; i < n; ++i) p.residual[i] = m[i];
        }
    }
    __syncthreads();
    for (int i = tid; i < p.width; i += kLaneThreads) {
        float acc = 0.0f;
        for (int lane = 0; lane < L; ++lane) acc = acc + gate_s[lane] * p.stream[(size_t)lane * p.width + i];
        p.input[i] = acc;
    }
}

__global__ __launch_bounds__(256) void lanes_combine_kernel(int lanes, int width, const float* post,
                                                            const float* residual, const float* stream,
                                                            const float* delta, float* next) {
    const int idx = blockIdx.x * kLaneThreads + threadIdx.x;
    if (idx >= lanes * width) return;
    const int lane = idx / width, i = idx - lane * width;
    float acc = 0.0f;
    for (int source = 0; source < lanes; ++source) acc = acc + residual[lane * lanes + source] * stream[(size_t)source * width + i];
    next[idx] = acc + post[lane] * delta[i];
}

hipError_t launch_lanes_prologue(const float* stream, int n, float* out, hipStream_t s) {
    if (n < 8 || n % 8 != 0) return hipErrorInvalidValue;
    rn_launch(lanes_prologue_kernel, dim3(1), dim3(kLaneThreads), 0, s, stream, n, out);
    return hipGetLastError();
}

hipError_t launch_lanes_route(const LanesRouteParams& p, hipStream_t s) {
    if (p.lanes < 1 || p.lanes > kMaxLanes || p.width < 1) return hipErrorInvalidValue;
    rn_launch(lanes_route_kernel, dim3(1), dim3(kLaneThreads), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_lanes_combine(int lanes, int width, const float* post, const float* residual, const float* stream,
                                const float* delta, float* next, hipStream_t s) {
    const long long n = (long long)lanes * width;
    if (lanes < 1 || width < 1) return hipErrorInvalidValue;
    rn_launch(lanes_combine_kernel, dim3((unsigned)((n + kLaneThreads - 1) / kLaneThreads)), dim3(kLaneThreads), 0, s,
              lanes, width, post, residual, stream, delta, next);
    return hipGetLastError();
}

}  // namespace rn
