// rn_misc.hip — small row kernels: per-row int8 quantisation (ops.rs:112-118),
// the zero-centred RMSNorm (ops.rs:44-50) with the eight-lane sum of squares of
// ops.rs:7-17, elementwise fast_exp / silu (ops.rs:73-90), the C library's expf
// and sigmoid over it (ops.rs:68-71), and the end of a
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
    const float inverse = reciprocal(sqrtf(mean_square + eps));
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
    peak = wave_max_nonneg(peak);
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

// op: 0 fast_exp, 1 silu, 2 the C library's expf, 3 sigmoid over it.
__global__ void fast_exp_kernel(const float* x, float* y, int n, int op) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    y[i] = op == 0 ? fast_exp(v) : op == 1 ? silu(v) : op == 2 ? libm_expf(v) : op == 3 ? libm_sigmoid(v)
                                   : op == 4 ? libm_logf(v) : reciprocal_normal(v);
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

hipError_t launch_fast_exp(const float* x, float* y, int n, int op, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    if (op < 0 || op > 5) return hipErrorInvalidValue;
    rn_launch(fast_exp_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, x, y, n, op);
    return hipGetLastError();
}

// QuantisedMatrix::dequantise_row (matrix.rs:140-153) for int8 codes: code x
// the scale of its group.
__global__ void dequantise_i8_kernel(const int8_t* codes, const float* scales, int columns, int group, float* out) {
    const int k = blockIdx.x * 256 + threadIdx.x;
    if (k < columns) out[k] = (float)codes[k] * scales[k / group];
}

hipError_t launch_dequantise_i8(const int8_t* codes, const float* scales, int columns, int group, float* out,
                                hipStream_t stream) {
    if (columns < 1 || group < 1) return hipErrorInvalidValue;
    rn_launch(dequantise_i8_kernel, dim3((columns + 255) / 256), dim3(256), 0, stream, codes, scales, columns, group,
              out);
    return hipGetLastError();
}

// kronecker_apply (ops.rs:166-217) for 32 x 32 factors, as the reference's
// aarch64 path computes it (ops.rs:220-297): one 1024-thread block per input
// [32][32]; thread (i, c) forms mixed[i][c] = sum over j of x[i][j] r[j][c]
// with fused multiply-adds in j order, then thread (k, c) out[k][c] = sum over
// i of l[i][k] mixed[i][c] with fused multiply-adds in i order. The input and
// both factors are staged in LDS.
__global__ __launch_bounds__(1024) void kronecker32_kernel(const float* input, const float* left, const float* right,
                                                           float* output) {
    __shared__ float x_s[1024], l_s[1024], r_s[1024], m_s[1024];
    const int t = threadIdx.x, row = t >> 5, col = t & 31;
    const float* x = input + (size_t)blockIdx.x * 1024;
    x_s[t] = x[t];
    l_s[t] = left[t];
    r_s[t] = right[t];
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) acc = fmaf(r_s[j * 32 + col], x_s[row * 32 + j], acc);
    m_s[t] = acc;
    __syncthreads();
    acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) acc = fmaf(m_s[i * 32 + col], l_s[i * 32 + row], acc);
    output[(size_t)blockIdx.x * 1024 + t] = acc;
}

hipError_t launch_kronecker32(const float* input, const float* left, const float* right, int count, float* output,
                              hipStream_t stream) {
    if (count < 0) return hipErrorInvalidValue;
    if (count == 0) return hipSuccess;
    rn_launch(kronecker32_kernel, dim3(count), dim3(1024), 0, stream, input, left, right, output);
    return hipGetLastError();
}

// The grammar-constrained choice of generator.rs:99-117 over n logits, one
// 1024-thread block.
//   1. Peaks (max is order-free: DPP within waves, then LDS), the greedy keys
//      of all and of allowed values (argmax_key: larger value, then lower
//      index) and the first allowed index. argmax_allowed (generator.rs:147-155)
//      is the first allowed index when its value is NaN, else the best allowed
//      key; with nothing allowed the choice falls back to argmax
//      (generator.rs:157-165).
//   2. allowed_statistics (generator.rs:182-194): the two totals are sequential
//      sums in index order, so the block computes fast_exp terms for 4096
//      values at a time into LDS and lanes 0 and 1 of wave 0 add them in order
//      (lane 0 the total over all values, lane 1 the allowed total, where a
//      disallowed term is multiplied by 0 as the reference does).
// token >= 0 asks for the statistics of that token instead of the choice.
__global__ __launch_bounds__(1024) void constrained_choice_kernel(const float* logits, const uint8_t* allowed, int n,
                                                                  int token, Choice* out) {
    constexpr int NT = 1024, NW = NT / 64, CH = 4096;
    __shared__ __align__(16) float ea_s[CH];
    __shared__ __align__(16) float ek_s[CH];
    __shared__ float pa_s[NW], pk_s[NW];
    __shared__ unsigned long long key_s[NW], akey_s[NW];
    __shared__ int first_s[NW];
    __shared__ float peaks_s[2];
    __shared__ int token_s, found_s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    float pa = -INFINITY, pk = -INFINITY;
    uint64_t key = 0, akey = 0;
    int first = n;
    for (int i = tid; i < n; i += NT) {
        const float v = logits[i];
        const bool ok = allowed[i] != 0;
        pa = fmaxf(pa, v);
        const uint64_t k = argmax_key(v, (uint32_t)i);
        key = k > key ? k : key;
        if (ok) {
            pk = fmaxf(pk, v);
            akey = k > akey ? k : akey;
            first = min(first, i);
        }
    }
    pa = wave_max(pa);
    pk = wave_max(pk);
    key = wave_max_u64(key);
    akey = wave_max_u64(akey);
    for (int o = 32; o >= 1; o >>= 1) first = min(first, __shfl_xor(first, o, 64));
    if (lane == 0) {
        pa_s[wave] = pa;
        pk_s[wave] = pk;
        key_s[wave] = key;
        akey_s[wave] = akey;
        first_s[wave] = first;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < NW; ++w) {
            pa = fmaxf(pa, pa_s[w]);
            pk = fmaxf(pk, pk_s[w]);
            key = key_s[w] > key ? key_s[w] : key;
            akey = akey_s[w] > akey ? akey_s[w] : akey;
            first = min(first, first_s[w]);
        }
        peaks_s[0] = pa;
        peaks_s[1] = pk;
        int t = token;
        const bool found = first < n;
        if (t < 0) {
            if (found)
                t = logits[first] != logits[first] ? first : (int)argmax_index(akey);
            else
                t = logits[0] != logits[0] ? 0 : (int)argmax_index(key);
        }
        token_s = t;
        found_s = found ? 1 : 0;
    }
    __syncthreads();
    const float peak_all = peaks_s[0], peak_allowed = peaks_s[1];

    float total = 0.0f;  // lane 0: over all values; lane 1: over allowed ones
    for (int base = 0; base < n; base += CH) {
        const int m = min(CH, n - base);
        for (int i = tid; i < m; i += NT) {
            const float v = logits[base + i];
            ea_s[i] = fast_exp(v - peak_all);
            ek_s[i] = fast_exp(v - peak_allowed) * (allowed[base + i] != 0 ? 1.0f : 0.0f);
        }
        __syncthreads();
        if (wave == 0 && lane < 2) {
            const float* src = lane == 0 ? ea_s : ek_s;
            int i = 0;
            for (; i + 4 <= m; i += 4) {
                const float4 q = *reinterpret_cast<const float4*>(src + i);
                total = total + q.x;
                total = total + q.y;
                total = total + q.z;
                total = total + q.w;
            }
            for (; i < m; ++i) total = total + src[i];
        }
        __syncthreads();
    }
    if (wave == 0) {
        const float total_allowed = __shfl(total, 1, 64);
        if (lane == 0) {
            const int t = token_s;
            Choice c;
            c.token = (uint32_t)t;
            c.constrained = found_s;
            c.probability = fast_exp(logits[t] - peak_allowed) / total_allowed;
            c.mass = (total_allowed * fast_exp(peak_allowed - peak_all)) / total;
            *out = c;
        }
    }
}

hipError_t launch_constrained_choice(const float* logits, const uint8_t* allowed, int n, int token, Choice* out,
                                     hipStream_t stream) {
    if (n < 1 || token >= n) return hipErrorInvalidValue;
    rn_launch(constrained_choice_kernel, dim3(1), dim3(1024), 0, stream, logits, allowed, n, token, out);
    return hipGetLastError();
}

}  // namespace rn
