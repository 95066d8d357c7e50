// rn_attention.hip — attention over a contiguous fp16 KV cache for gfx950.
//
// Replaces AttentionWeights::attend / attend_heads (crates/model/src/attention.rs:
// 96-213) and kernels::attend_head (crates/kernels/src/attention.rs:251-280) for
// an fp16 cache: score = q.k / sqrt(head_dim), peak-subtracted fast_exp weights,
// weighted values, one multiply by 1/total.
//
// One 256-thread block per (head, query). The block is sixteen 16-lane groups:
// group gi takes positions gi, gi+16, ... and lane li of a group owns dims
// 4li..4li+3, so one 16-lane group reads one 128-byte cache row and a wave reads
// four consecutive rows. The float reductions follow the fixed trees:
//   score (T2): 0 + q0k0 + ... + q3k3 per lane, then a balanced butterfly
//               (xor 1, 2, 4, 8) across the 16 lanes;
//   total and P.V (T3): the per-group running sums over positions gi, gi+16, ...
//               (increasing), then groups 0..15 added in order.
// Scores live in LDS (dynamic, one float per position).
#include "rn_device.hpp"
#include "rn_internal.hpp"

namespace rn {

constexpr int kHeadDim = 64;
constexpr int kLanesPerRow = 16;
constexpr int kPer = kHeadDim / kLanesPerRow;  // 4 dims per lane
constexpr int kGroups = 256 / kLanesPerRow;     // 16 position groups

__device__ __forceinline__ void load4(const __half* row, int li, float* out) {
    const uint2 raw = *reinterpret_cast<const uint2*>(row + li * kPer);
    const __half2 a = *reinterpret_cast<const __half2*>(&raw.x);
    const __half2 b = *reinterpret_cast<const __half2*>(&raw.y);
    out[0] = __low2float(a);
    out[1] = __high2float(a);
    out[2] = __low2float(b);
    out[3] = __high2float(b);
}

template <int MODE>
__global__ __launch_bounds__(256) void attend_kernel(AttendParams p) {
    extern __shared__ float scores[];
    __shared__ float q_s[kHeadDim];
    __shared__ float part_s[kGroups][kHeadDim];
    __shared__ float total_s[kGroups];
    __shared__ float peak_s[4];

    const int tid = threadIdx.x;
    const int gi = tid / kLanesPerRow;
    const int li = tid % kLanesPerRow;

    const __half* K;
    const __half* V;
    float* out;
    int length;

    if constexpr (MODE == kAttendDecode) {
        const int h = blockIdx.x, b = blockIdx.y;
        const int pos = p.pos[(size_t)b * p.pos_stride];
        if (pos < 0 || pos >= p.capacity) {
            if (tid == 0) atomicOr(p.error, 2);
            return;
        }
        length = pos + 1;
        const size_t base = (size_t)b * p.seq_stride + ((size_t)p.layer * p.heads + h) * p.capacity * kHeadDim;
        __half* Kw = p.kc + base;
        __half* Vw = p.vc + base;
        K = Kw;
        V = Vw;
        out = p.out + (size_t)b * p.d_model + h * kHeadDim;
        const float* row = p.qkv + (size_t)b * 3 * p.d_model;
        if (tid < kHeadDim / 2) {  // ops.rs:131-141 rotate-half at `pos`, then the fp16 append
            const int i = tid, half = kHeadDim / 2;
            const float c = p.rope_cos[(size_t)pos * half + i];
            const float s = p.rope_sin[(size_t)pos * half + i];
            const float qa = row[h * kHeadDim + i], qb = row[h * kHeadDim + i + half];
            q_s[i] = qa * c - qb * s;
            q_s[i + half] = qb * c + qa * s;
            const float ka = row[p.d_model + h * kHeadDim + i], kb = row[p.d_model + h * kHeadDim + i + half];
            Kw[(size_t)pos * kHeadDim + i] = __float2half_rn(ka * c - kb * s);
            Kw[(size_t)pos * kHeadDim + i + half] = __float2half_rn(kb * c + ka * s);
            Vw[(size_t)pos * kHeadDim + i] = __float2half_rn(row[2 * p.d_model + h * kHeadDim + i]);
            Vw[(size_t)pos * kHeadDim + i + half] = __float2half_rn(row[2 * p.d_model + h * kHeadDim + i + half]);
        }
    } else if constexpr (MODE == kAttendPrefill) {
        const int h = blockIdx.x, t = blockIdx.y;
        length = p.first + t + 1;
        const size_t base = ((size_t)p.layer * p.heads + h) * p.capacity * kHeadDim;
        K = p.kc + base;
        V = p.vc + base;
        out = p.out + (size_t)t * p.d_model + h * kHeadDim;
        if (tid < kHeadDim) q_s[tid] = p.q[(size_t)t * p.d_model + h * kHeadDim + tid];
    } else {
        const int i = blockIdx.x;
        length = p.lengths[i];
        if (length < 1 || length > p.stride) {
            if (tid == 0) atomicOr(p.error, 4);
            return;
        }
        K = p.kc + (size_t)i * p.stride * kHeadDim;
        V = p.vc + (size_t)i * p.stride * kHeadDim;
        out = p.out + (size_t)i * kHeadDim;
        if (tid < kHeadDim) q_s[tid] = p.q[(size_t)i * kHeadDim + tid];
    }
    __syncthreads();  // q_s, and the appended row is visible to the whole block

    // scores (T2), four positions in flight per group
    const float inverse_root = 1.0f / sqrtf((float)kHeadDim);
    float q4[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) q4[i] = q_s[li * kPer + i];
    for (int p0 = 0; p0 < length; p0 += 4 * kGroups) {
        float k4[4][kPer];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int pp = p0 + u * kGroups + gi;
            if (pp < length)
                load4(K + (size_t)pp * kHeadDim, li, k4[u]);
            else
#pragma unroll
                for (int i = 0; i < kPer; ++i) k4[u][i] = 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < kPer; ++i) s = s + q4[i] * k4[u][i];
            s = s + __shfl_xor(s, 1, kLanesPerRow);
            s = s + __shfl_xor(s, 2, kLanesPerRow);
            s = s + __shfl_xor(s, 4, kLanesPerRow);
            s = s + __shfl_xor(s, 8, kLanesPerRow);
            const int pp = p0 + u * kGroups + gi;
            if (li == 0 && pp < length) scores[pp] = s * inverse_root;
        }
    }
    __syncthreads();

    // peak (order-free) and the fast_exp weights
    float m = -INFINITY;
    for (int pp = tid; pp < length; pp += 256) m = fmaxf(m, scores[pp]);
    m = wave_max(m);
    if ((tid & 63) == 0) peak_s[tid >> 6] = m;
    __syncthreads();
    const float peak = fmaxf(fmaxf(peak_s[0], peak_s[1]), fmaxf(peak_s[2], peak_s[3]));
    for (int pp = tid; pp < length; pp += 256) scores[pp] = fast_exp(scores[pp] - peak);
    __syncthreads();

    // weighted values (T3)
    float acc[kPer] = {0.0f, 0.0f, 0.0f, 0.0f};
    float total = 0.0f;
    for (int p0 = gi; p0 < length; p0 += 4 * kGroups) {
        float v4[4][kPer];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int pp = p0 + u * kGroups;
            if (pp < length) load4(V + (size_t)pp * kHeadDim, li, v4[u]);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int pp = p0 + u * kGroups;
            if (pp < length) {
                const float e = scores[pp];
#pragma unroll
                for (int i = 0; i < kPer; ++i) acc[i] = acc[i] + e * v4[u][i];
                total = total + e;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) part_s[gi][li * kPer + i] = acc[i];
    if (li == 0) total_s[gi] = total;
    __syncthreads();
    if (tid < kHeadDim) {
        float o = 0.0f, t = 0.0f;
#pragma unroll
        for (int j = 0; j < kGroups; ++j) {
            o = o + part_s[j][tid];
            t = t + total_s[j];
        }
        const float inverse = 1.0f / t;
        out[tid] = o * inverse;
    }
}

hipError_t launch_attend(const AttendParams& p, int mode, int grid_x, int grid_y, int max_length,
                         hipStream_t stream) {
    const size_t lds = sizeof(float) * (size_t)(max_length > 0 ? max_length : 1);
    if (lds > 96 * 1024) return hipErrorInvalidValue;
    const dim3 grid(grid_x, grid_y);
    switch (mode) {
        case kAttendDecode:
            hipLaunchKernelGGL(attend_kernel<kAttendDecode>, grid, dim3(256), lds, stream, p);
            break;
        case kAttendPrefill:
            hipLaunchKernelGGL(attend_kernel<kAttendPrefill>, grid, dim3(256), lds, stream, p);
            break;
        case kAttendRaw:
            hipLaunchKernelGGL(attend_kernel<kAttendRaw>, grid, dim3(256), lds, stream, p);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Prefill rotary + append: one block per token, one thread per (head, pair).
__global__ __launch_bounds__(256) void rope_append_kernel(const float* qkv, float* q_out, __half* kc, __half* vc,
                                                          int layer, int heads, int capacity, int d_model, int first,
                                                          const float* rope_cos, const float* rope_sin) {
    const int t = blockIdx.x;
    const int half = kHeadDim / 2;
    const int pos = first + t;
    const float* row = qkv + (size_t)t * 3 * d_model;
    for (int idx = threadIdx.x; idx < heads * half; idx += blockDim.x) {
        const int h = idx / half, i = idx % half;
        const float c = rope_cos[(size_t)pos * half + i];
        const float s = rope_sin[(size_t)pos * half + i];
        const float qa = row[h * kHeadDim + i], qb = row[h * kHeadDim + i + half];
        q_out[(size_t)t * d_model + h * kHeadDim + i] = qa * c - qb * s;
        q_out[(size_t)t * d_model + h * kHeadDim + i + half] = qb * c + qa * s;
        const size_t base = (((size_t)layer * heads + h) * capacity + pos) * kHeadDim;
        const float ka = row[d_model + h * kHeadDim + i], kb = row[d_model + h * kHeadDim + i + half];
        kc[base + i] = __float2half_rn(ka * c - kb * s);
        kc[base + i + half] = __float2half_rn(kb * c + ka * s);
        vc[base + i] = __float2half_rn(row[2 * d_model + h * kHeadDim + i]);
        vc[base + i + half] = __float2half_rn(row[2 * d_model + h * kHeadDim + i + half]);
    }
}

hipError_t launch_rope_append(const float* qkv, float* q_out, __half* kc, __half* vc, int layer, int heads,
                              int capacity, int d_model, int first, int count, const float* rope_cos,
                              const float* rope_sin, hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    hipLaunchKernelGGL(rope_append_kernel, dim3(count), dim3(256), 0, stream, qkv, q_out, kc, vc, layer, heads,
                       capacity, d_model, first, rope_cos, rope_sin);
    return hipGetLastError();
}

}  // namespace rn
