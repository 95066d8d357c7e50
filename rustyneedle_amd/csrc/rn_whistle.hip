// rn_whistle.hip — the speech path's own kernels for gfx950: the fp32 stem
// convolutions, per-head norm/rotary/int8 codes, attention with int8 queries,
// keys and values, and the cross-attention residual.
//
// Replaces crates/whistle/src/stem.rs:39-115 (first convolution, one
// depthwise + pointwise stage), encoder.rs:217-297 (the attention's integer
// scores and int8 values) and cross.rs:58-182 (memory, apply). Products go
// through the shared int8 kernels (rn_gemm.hip, rn_gemv.hip).
//
// Float orders (identical to the CPU restatement): the first convolution adds
// its taps (k, m) in order into a zero output per (frame, channel); the
// depthwise convolution adds its three taps in order; the head norm uses the
// eight-lane sum of ops.rs:7-17; softmax totals and value sums use 32
// interleaved frame classes (frame j goes to class j mod 32, classes summed
// 0..31), with the weights normalised first and scaled by the value scale
// (ops.rs:92-101, encoder.rs:278-285).
#include "rn_device.hpp"
#include "rn_internal.hpp"

namespace rn {

constexpr int kStemTime = 32;   // output frames per block of the first convolution
constexpr int kStemChan = 32;   // channels per block
constexpr int kMaxMels = 128;

// stem.rs:44-62 in one dimension of time: out[t][c] = silu(sum over taps (k, m)
// of mel[t + k - 1][m] * w[c][k][m]), frames outside [0, F) skipped.
__global__ __launch_bounds__(256) void stem_conv_kernel(const float* mel, const float* w, int F, int M, int d,
                                                        float* out) {
    extern __shared__ float lds[];
    const int WS = 3 * M + 1;                  // padded weight row: distinct banks per channel
    float* w_s = lds;                          // [kStemChan][WS]
    float* x_s = lds + kStemChan * WS;         // [kStemTime + 2][M]
    const int t0 = blockIdx.x * kStemTime, c0 = blockIdx.y * kStemChan;
    for (int i = threadIdx.x; i < kStemChan * 3 * M; i += 256) {
        const int c = i / (3 * M), r = i - c * 3 * M;
        w_s[c * WS + r] = w[(size_t)min(c0 + c, d - 1) * 3 * M + r];
    }
    for (int i = threadIdx.x; i < (kStemTime + 2) * M; i += 256) {
        const int r = i / M, m = i - r * M;
        const int src = t0 + r - 1;
        x_s[i] = (src >= 0 && src < F) ? mel[(size_t)src * M + m] : 0.0f;
    }
    __syncthreads();
    const int c = threadIdx.x & 31, tg = threadIdx.x >> 5;  // 32 channels x 8 frame groups
    const float* wr = w_s + c * WS;
    for (int i = 0; i < kStemTime / 8; ++i) {
        const int tl = tg + 8 * i, t = t0 + tl;
        float acc = 0.0f;
        for (int k = 0; k < 3; ++k) {
            const int src = t + k - 1;
            if (src < 0 || src >= F) continue;
            const float* xr = x_s + (tl + k) * M;
            const float* wk = wr + k * M;
            for (int m = 0; m < M; ++m) acc = acc + xr[m] * wk[m];
        }
        if (t < F && c0 + c < d) out[(size_t)t * d + c0 + c] = silu(acc);
    }
}

// stem.rs:64-94, the stage's depthwise convolution (kernel 3, stride 2, pad 1).
__global__ __launch_bounds__(256) void stem_depthwise_kernel(const float* h, const float* dw, int F, int T, int d,
                                                             float* out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= T * d) return;
    const int t = i / d, c = i - t * d;
    float acc = 0.0f;
    for (int k = 0; k < 3; ++k) {
        const int src = 2 * t + k - 1;
        if (src < 0 || src >= F) continue;
        acc = acc + h[(size_t)src * d + c] * dw[(size_t)k * d + c];
    }
    out[i] = acc;
}

hipError_t launch_stem(const float* mel, const float* conv1, const float* depthwise, int F, int M, int d, float* h1,
                       float* dw_out, hipStream_t stream) {
    if (M < 1 || M > kMaxMels || F < 1 || d < 1) return hipErrorInvalidValue;
    const int T = (F - 1) / 2 + 1;
    const size_t lds = sizeof(float) * ((size_t)kStemChan * (3 * M + 1) + (size_t)(kStemTime + 2) * M);
    rn_launch(stem_conv_kernel, dim3((F + kStemTime - 1) / kStemTime, (d + kStemChan - 1) / kStemChan), dim3(256), lds,
              stream, mel, conv1, F, M, d, h1);
    rn_launch(stem_depthwise_kernel, dim3((T * d + 255) / 256), dim3(256), 0, stream, h1, depthwise, F, T, d, dw_out);
    return hipGetLastError();
}

// Per-(frame, head, section) int8 codes of one 64-dim head, one wave each:
// optional zero-centred norm with the head gains (ops.rs:44-50; lane j < 8 of
// the eight-lane sum gathers elements j, j+8, ... by shuffles), optional
// rotate-half rotary at the frame's position (ops.rs:131-141), then
// quantise_int8; the stored scale is multiplied by the section's factor
// (1/sqrt(head_dim) for queries, encoder.rs:239-244, 270).
__global__ __launch_bounds__(256) void head_codes_kernel(HeadCodesParams p) {
    const int wave = (blockIdx.x * 256 + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    const int per_frame = p.heads * p.nsec;
    const bool live = wave < p.frames * per_frame;
    const int w = live ? wave : 0;
    const int t = w / per_frame, r = w - t * per_frame;
    const int si = r / p.heads, h = r - si * p.heads;
    const HeadSection& sec = p.sec[si];
    float v = p.src[(size_t)t * p.src_stride + sec.col + h * 64 + lane];
    if (sec.gain != nullptr) {
        const float sq = v * v;
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) s = s + __shfl(sq, 8 * c + (lane & 7), kWave);
        float total = sum_lanes_0_to_7(s);
        total = total + 0.0f;
        const float inverse = 1.0f / sqrtf(total / 64.0f + p.eps);
        v = ((1.0f + sec.gain[lane]) * v) * inverse;
    }
    if (sec.rotary) {
        const int pos = p.pos0 + t, i = lane & 31;
        const float c = p.rope_cos[(size_t)pos * 32 + i], s = p.rope_sin[(size_t)pos * 32 + i];
        const float other = __shfl_xor(v, 32, kWave);
        v = lane < 32 ? v * c - other * s : v * c + other * s;
    }
    const float peak = wave_max(fabsf(v));
    const float scale = int8_scale_from_peak(peak);
    float y;
    quotients<1>(&v, scale, &y);
    if (!live) return;
    sec.codes[((size_t)t * p.heads + h) * 64 + lane] = (int8_t)code_of_quotient(y);
    if (lane == 0) sec.scales[(size_t)t * p.heads + h] = scale * sec.scale_mul;
}

hipError_t launch_head_codes(const HeadCodesParams& p, hipStream_t stream) {
    const long waves = (long)p.frames * p.heads * p.nsec;
    if (waves <= 0) return hipSuccess;
    rn_launch(head_codes_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream, p);
    return hipGetLastError();
}

// One (query, head) per 256-thread block over `frames` int8 key/value rows.
// Scores ((float)dot * key_scale) * query_scale in LDS (dynamic: one float per
// frame), the peak, fast_exp, class totals (thread c sums frames c, c+32, ...
// in order), the weights value_scale * (e * (1 / total)), then thread
// (class c, dims 8g..8g+7) sums its class's weighted value codes in frame
// order and the classes are added 0..31.
__global__ __launch_bounds__(256) void int8_attend_kernel(Int8AttendParams p) {
    extern __shared__ float e_s[];
    __shared__ float part_s[32][65];
    __shared__ float tot_s[32];
    __shared__ float peak_s[4];
    const int q = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int F = p.frames, H = p.heads;
    const int4* qrow = reinterpret_cast<const int4*>(p.qc + ((size_t)q * H + h) * 64);
    const int4 q0 = qrow[0], q1 = qrow[1], q2 = qrow[2], q3 = qrow[3];
    const float qs = p.qs[(size_t)q * H + h];
    float m = -INFINITY;
    for (int j = tid; j < F; j += 256) {
        const int4* krow = reinterpret_cast<const int4*>(p.kc + ((size_t)j * H + h) * 64);
        int dot = dot16(krow[0], q0, 0);
        dot = dot16(krow[1], q1, dot);
        dot = dot16(krow[2], q2, dot);
        dot = dot16(krow[3], q3, dot);
        const float s = ((float)dot * p.ks[(size_t)j * H + h]) * qs;
        e_s[j] = s;
        m = fmaxf(m, s);
    }
    m = wave_max(m);
    if ((tid & 63) == 0) peak_s[tid >> 6] = m;
    __syncthreads();
    const float peak = fmaxf(fmaxf(peak_s[0], peak_s[1]), fmaxf(peak_s[2], peak_s[3]));
    for (int j = tid; j < F; j += 256) e_s[j] = fast_exp(e_s[j] - peak);
    __syncthreads();
    if (tid < 32) {
        float t = 0.0f;
        for (int j = tid; j < F; j += 32) t = t + e_s[j];
        tot_s[tid] = t;
    }
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int c = 0; c < 32; ++c) total = total + tot_s[c];
    const float inverse = 1.0f / total;
    __syncthreads();  // every thread has read the class totals
    for (int j = tid; j < F; j += 256) e_s[j] = p.vs[(size_t)j * H + h] * (e_s[j] * inverse);
    __syncthreads();
    const int c = tid >> 3, g = tid & 7;
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = c; j < F; j += 32) {
        const int2 raw = *reinterpret_cast<const int2*>(p.vc + ((size_t)j * H + h) * 64 + 8 * g);
        const float wj = e_s[j];
        const int8_t* b = reinterpret_cast<const int8_t*>(&raw);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = acc[i] + wj * (float)b[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) part_s[c][8 * g + i] = acc[i];
    __syncthreads();
    if (tid < 64) {
        float o = 0.0f;
#pragma unroll
        for (int k = 0; k < 32; ++k) o = o + part_s[k][tid];
        p.out[(size_t)q * p.out_stride + h * 64 + tid] = o;
    }
}

hipError_t launch_int8_attend(const Int8AttendParams& p, int queries, hipStream_t stream) {
    if (queries <= 0) return hipSuccess;
    const size_t lds = sizeof(float) * (size_t)(p.frames > 0 ? p.frames : 1);
    if (p.frames < 1 || lds > 128 * 1024) return hipErrorInvalidValue;
    rn_launch(int8_attend_kernel, dim3(queries, p.heads), dim3(256), lds, stream, p);
    return hipGetLastError();
}

// cross.rs:176-181: x += gain * zero_centred_norm(attended, post_norm), one
// wave over the whole vector (E values per lane).
template <int E>
__global__ __launch_bounds__(64) void cross_residual_kernel(const float* attended, const float* gain_vec, float gain,
                                                           float eps, float* x) {
    constexpr int n = 64 * E;
    __shared__ float sq_s[n];
    const int lane = threadIdx.x;
    float v[E];
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = attended[lane * E + e];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int idx = lane * E + e;
        sq_s[(idx % 8) * (n / 8) + idx / 8] = v[e] * v[e];
    }
    __syncthreads();
    float s = 0.0f;
    if (lane < 8)
        for (int c = 0; c < n / 8; ++c) s = s + sq_s[lane * (n / 8) + c];
    float total = sum_lanes_0_to_7(s);
    total = total + 0.0f;
    const float inverse = 1.0f / sqrtf(total / (float)n + eps);
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int idx = lane * E + e;
        const float normed = ((1.0f + gain_vec[idx]) * v[e]) * inverse;
        x[idx] = x[idx] + gain * normed;
    }
}

hipError_t launch_cross_residual(const float* attended, const float* post_norm, float gain, float eps, int n, float* x,
                                 hipStream_t stream) {
    switch (n) {
        case 384:
            rn_launch(cross_residual_kernel<6>, dim3(1), dim3(64), 0, stream, attended, post_norm, gain, eps, x);
            break;
        case 512:
            rn_launch(cross_residual_kernel<8>, dim3(1), dim3(64), 0, stream, attended, post_norm, gain, eps, x);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

__global__ void add_rows_kernel(const float* a, const float* b, size_t n, float* out) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

hipError_t launch_add(const float* a, const float* b, size_t n, float* out, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    rn_launch(add_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a, b, n, out);
    return hipGetLastError();
}

}  // namespace rn
