// rn_misc.hip — small row kernels: per-row int8 quantisation (ops.rs:112-118),
// the zero-centred RMSNorm (ops.rs:44-50) with the eight-lane sum of squares of
// ops.rs:7-17, elementwise fast_exp / silu (ops.rs:73-90), and the end of a
// push (final norm into the session's hidden state, position advance).
#include "rn_device.hpp"
#include "rn_internal.hpp"

namespace rn {

LaunchEvents& launch_events() {
    static thread_local LaunchEvents events;
    return events;
}

constexpr int kRowThreads = 64;
constexpr int kMaxRow = 4096;

// Zero-centred norm of one row held in LDS `v` (n values), written to `out`.
// Lanes 0..7 of the wave run the eight strided partial sums of ops.rs:7-17.
__device__ void norm_row(const float* v, const float* gain, int n, float eps, float* out, float* lanes_s) {
    const int lane = threadIdx.x;
    if (lane < 8) {
        float s = 0.0f;
        for (int c = 0; c < n / 8; ++c) {
            const float x = v[8 * c + lane];
            s = s + x * x;
        }
        lanes_s[lane] = s;
    }
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) total = total + lanes_s[j];
    total = total + 0.0f;
    const float mean_square = total / (float)n;
    const float inverse = 1.0f / sqrtf(mean_square + eps);
    for (int i = lane; i < n; i += kRowThreads) out[i] = ((1.0f + gain[i]) * v[i]) * inverse;
}

__global__ __launch_bounds__(64) void norm_rows_kernel(const float* x, const float* gain, int n, float eps,
                                                       float* out) {
    __shared__ float v[kMaxRow];
    __shared__ float lanes_s[8];
    const float* row = x + (size_t)blockIdx.x * n;
    for (int i = threadIdx.x; i < n; i += kRowThreads) v[i] = row[i];
    __syncthreads();
    norm_row(v, gain, n, eps, out + (size_t)blockIdx.x * n, lanes_s);
}

__global__ __launch_bounds__(64) void finish_push_kernel(const float* x, const float* gain, int n, float eps,
                                                         float* hidden, DecodeState* state) {
    __shared__ float v[kMaxRow];
    __shared__ float lanes_s[8];
    for (int i = threadIdx.x; i < n; i += kRowThreads) v[i] = x[i];
    __syncthreads();
    norm_row(v, gain, n, eps, hidden, lanes_s);
    if (threadIdx.x == 0) state->pos = state->pos + 1;
}

__global__ __launch_bounds__(64) void quantise_rows_kernel(const float* x, int n, int8_t* codes, float* scales) {
    const float* row = x + (size_t)blockIdx.x * n;
    float peak = 0.0f;
    for (int i = threadIdx.x; i < n; i += kRowThreads) peak = fmaxf(peak, fabsf(row[i]));
    peak = wave_max(peak);
    const float scale = int8_scale_from_peak(peak);
    for (int i0 = 0; i0 < n; i0 += kRowThreads) {  // uniform trip count: every lane reaches the wave vote
        const int i = i0 + threadIdx.x;
        const float v = i < n ? row[i] : 0.0f;
        float y;
        quotients<1>(&v, scale, &y);
        if (i < n) codes[(size_t)blockIdx.x * n + i] = (int8_t)code_of_quotient(y);
    }
    if (threadIdx.x == 0) scales[blockIdx.x] = scale;
}

__global__ void fast_exp_kernel(const float* x, float* y, int n, int apply_silu) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = apply_silu ? silu(x[i]) : fast_exp(x[i]);
}

hipError_t launch_norm_rows(const float* x, const float* gain, int count, int n, float eps, float* out,
                            hipStream_t stream) {
    if (n % 8 != 0 || n > kMaxRow || n <= 0) return hipErrorInvalidValue;
    if (count <= 0) return hipSuccess;
    rn_launch(norm_rows_kernel, dim3(count), dim3(kRowThreads), 0, stream, x, gain, n, eps, out);
    return hipGetLastError();
}

hipError_t launch_finish_push(const float* x, const float* gain, int n, float eps, float* hidden,
                              DecodeState* state, hipStream_t stream) {
    if (n % 8 != 0 || n > kMaxRow) return hipErrorInvalidValue;
    rn_launch(finish_push_kernel, dim3(1), dim3(kRowThreads), 0, stream, x, gain, n, eps, hidden, state);
    return hipGetLastError();
}

hipError_t launch_quantise_rows(const float* x, int count, int columns, int8_t* codes, float* scales,
                                hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    rn_launch(quantise_rows_kernel, dim3(count), dim3(kRowThreads), 0, stream, x, columns, codes, scales);
    return hipGetLastError();
}

__global__ void set_state_kernel(DecodeState* st, uint32_t token, int32_t pos, uint32_t step, uint32_t ids_capacity) {
    st->token = token;
    st->pos = pos;
    st->step = step;
    st->ids_capacity = ids_capacity;
}

hipError_t launch_set_state(DecodeState* state, uint32_t token, int32_t pos, uint32_t step, uint32_t ids_capacity,
                            hipStream_t stream) {
    rn_launch(set_state_kernel, dim3(1), dim3(1), 0, stream, state, token, pos, step, ids_capacity);
    return hipGetLastError();
}

hipError_t launch_fast_exp(const float* x, float* y, int n, int apply_silu, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    rn_launch(fast_exp_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, x, y, n, apply_silu);
    return hipGetLastError();
}

}  // namespace rn
