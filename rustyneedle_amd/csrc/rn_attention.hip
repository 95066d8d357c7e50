// rn_attention.hip — attention over a contiguous fp16 KV cache for gfx950.
//
// Replaces AttentionWeights::attend / attend_heads (crates/model/src/attention.rs:
// 96-213) and kernels::attend_head (crates/kernels/src/attention.rs:251-280) for
// an fp16 cache: score = q.k / sqrt(head_dim), peak-subtracted fast_exp weights,
// weighted values, one multiply by 1/total.
//
// One 256-thread block per (head, query). Latency is the enemy at these sizes
// (a head's cache is 2 x L x 128 bytes), so every cache load that does not
// depend on the current token is issued before anything else: the first chunk
// of key rows (up to 384 positions) and of value rows goes out at once, and
// only then does the block read its q/k/v row, apply the rotary and append the
// new key/value. The new position is served from LDS.
//
// Scores: 8 lanes per key row, 16 bytes (8 dims) each; a wave covers 8 rows per
// load, the block 32 rows per pass. Values: 16 lanes per row, 8 bytes (4 dims)
// each; thread (j, dg) walks positions j, j+16, j+32, ... The float reductions
// follow the fixed trees of the CPU restatement:
//   score (T2): per 4 dims 0 + q0k0 + ... + q3k3; the 16 sub-sums combined by a
//               balanced pairwise tree (the first level inside a lane, then
//               xor 1, 2, 4 across the 8 lanes);
//   total and P.V (T3): sixteen running sums over positions j, j+16, ... in
//               increasing order, then added j = 0..15.
// Scores live in LDS (dynamic, one float per position).
#include "rn_device.hpp"
#include "rn_internal.hpp"

namespace rn {

constexpr int kHeadDim = 64;
constexpr int kKChunk = 12;   // key passes of 32 rows issued together (384 positions)
constexpr int kVChunk = 24;   // value positions per thread issued together (384 positions)

__device__ __forceinline__ void unpack8(const uint4& raw, float* out) {
    const __half2* h = reinterpret_cast<const __half2*>(&raw);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[2 * i] = __low2float(h[i]);
        out[2 * i + 1] = __high2float(h[i]);
    }
}

__device__ __forceinline__ void unpack4(const uint2& raw, float* out) {
    const __half2* h = reinterpret_cast<const __half2*>(&raw);
    out[0] = __low2float(h[0]);
    out[1] = __high2float(h[0]);
    out[2] = __low2float(h[1]);
    out[3] = __high2float(h[1]);
}

// T2 for one key row held as 8 dims per lane (lane li owns dims 8li..8li+7).
__device__ __forceinline__ float score_row(const float* q8, const float* k8) {
    float a = 0.0f, b = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) a = a + q8[i] * k8[i];
#pragma unroll
    for (int i = 4; i < 8; ++i) b = b + q8[i] * k8[i];
    float s = a + b;
    s = s + __shfl_xor(s, 1, 8);
    s = s + __shfl_xor(s, 2, 8);
    s = s + __shfl_xor(s, 4, 8);
    return s;
}

template <int MODE>
__global__ __launch_bounds__(256) void attend_kernel(AttendParams p) {
    extern __shared__ float scores[];
    __shared__ float q_s[kHeadDim];
    __shared__ __align__(16) __half new_s[2][kHeadDim];  // decode: the appended key and value
    __shared__ float part_s[16][kHeadDim];
    __shared__ float total_s[16];
    __shared__ float peak_s[4];

    const int tid = threadIdx.x;
    const int r = tid >> 3, li = tid & 7;    // score layout: row slot, 8-dim lane
    const int j = tid >> 4, dg = tid & 15;   // value layout: position class, 4-dim lane

    const __half* K;
    const __half* V;
    float* out;
    int nglobal;     // positions read from the cache in global memory
    bool has_new;    // decode: one more position (index nglobal) served from LDS
    int pos = 0;

    if constexpr (MODE == kAttendDecode) {
        const int h = blockIdx.x, b = blockIdx.y;
        pos = p.pos[(size_t)b * p.pos_stride];
        if (pos < 0 || pos >= p.capacity) {
            if (tid == 0) atomicOr(p.error, 2);
            return;
        }
        const size_t base = (size_t)b * p.seq_stride + ((size_t)p.layer * p.heads + h) * p.capacity * kHeadDim;
        K = p.kc + base;
        V = p.vc + base;
        out = p.out + (size_t)b * p.d_model + h * kHeadDim;
        nglobal = pos;
        has_new = true;
    } else if constexpr (MODE == kAttendPrefill) {
        const int h = blockIdx.x, t = blockIdx.y;
        const size_t base = ((size_t)p.layer * p.heads + h) * p.capacity * kHeadDim;
        K = p.kc + base;
        V = p.vc + base;
        out = p.out + (size_t)t * p.d_model + h * kHeadDim;
        nglobal = p.first + t + 1;
        has_new = false;
    } else {
        const int i = blockIdx.x;
        const int length = p.lengths[i];
        if (length < 1 || length > p.stride) {
            if (tid == 0) atomicOr(p.error, 4);
            return;
        }
        K = p.kc + (size_t)i * p.stride * kHeadDim;
        V = p.vc + (size_t)i * p.stride * kHeadDim;
        out = p.out + (size_t)i * kHeadDim;
        nglobal = length;
        has_new = false;
    }
    const int length = nglobal + (has_new ? 1 : 0);
    // Loads past the last cached row re-read it (always inside the cache); their
    // results are discarded by selects, never by branches, so no branch splits
    // the load stream and forces a full wait.
    const int last = nglobal > 0 ? nglobal - 1 : 0;

    // 1. cache loads that do not depend on the current token, issued first
    uint4 kr[kKChunk];
#pragma unroll
    for (int c = 0; c < kKChunk; ++c) {
        const int pp = r + 32 * c;
        kr[c] = *reinterpret_cast<const uint4*>(K + (size_t)min(pp, last) * kHeadDim + 8 * li);
    }
    uint2 vr[kVChunk];
#pragma unroll
    for (int c = 0; c < kVChunk; ++c) {
        const int pp = j + 16 * c;
        vr[c] = *reinterpret_cast<const uint2*>(V + (size_t)min(pp, last) * kHeadDim + 4 * dg);
    }

    // 2. the query (and, when decoding, the rotary + fp16 append of the new row)
    if constexpr (MODE == kAttendDecode) {
        const int h = blockIdx.x, b = blockIdx.y;
        const float* row = p.qkv + (size_t)b * 3 * p.d_model;
        if (tid < kHeadDim / 2) {  // ops.rs:131-141 rotate-half at `pos`
            const int i = tid, half = kHeadDim / 2;
            const float c = p.rope_cos[(size_t)pos * half + i];
            const float s = p.rope_sin[(size_t)pos * half + i];
            const float qa = row[h * kHeadDim + i], qb = row[h * kHeadDim + i + half];
            q_s[i] = qa * c - qb * s;
            q_s[i + half] = qb * c + qa * s;
            const float ka = row[p.d_model + h * kHeadDim + i], kb = row[p.d_model + h * kHeadDim + i + half];
            const __half k0 = __float2half_rn(ka * c - kb * s), k1 = __float2half_rn(kb * c + ka * s);
            const __half v0 = __float2half_rn(row[2 * p.d_model + h * kHeadDim + i]);
            const __half v1 = __float2half_rn(row[2 * p.d_model + h * kHeadDim + i + half]);
            new_s[0][i] = k0;
            new_s[0][i + half] = k1;
            new_s[1][i] = v0;
            new_s[1][i + half] = v1;
            __half* Kw = const_cast<__half*>(K) + (size_t)pos * kHeadDim;
            __half* Vw = const_cast<__half*>(V) + (size_t)pos * kHeadDim;
            Kw[i] = k0;
            Kw[i + half] = k1;
            Vw[i] = v0;
            Vw[i + half] = v1;
        }
    } else if constexpr (MODE == kAttendPrefill) {
        if (tid < kHeadDim) q_s[tid] = p.q[(size_t)blockIdx.y * p.d_model + blockIdx.x * kHeadDim + tid];
    } else {
        if (tid < kHeadDim) q_s[tid] = p.q[(size_t)blockIdx.x * kHeadDim + tid];
    }
    __syncthreads();

    // 3. scores (T2)
    const float inverse_root = 1.0f / sqrtf((float)kHeadDim);
    float q8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) q8[i] = q_s[8 * li + i];
    for (int base = 0; base < nglobal; base += 32 * kKChunk) {
        if (base > 0) {
#pragma unroll
            for (int c = 0; c < kKChunk; ++c) {
                const int pp = base + r + 32 * c;
                kr[c] = *reinterpret_cast<const uint4*>(K + (size_t)min(pp, last) * kHeadDim + 8 * li);
            }
        }
#pragma unroll
        for (int c = 0; c < kKChunk; ++c) {
            const int pp = base + r + 32 * c;
            float k8[8];
            unpack8(kr[c], k8);
            const float s = score_row(q8, k8);
            if (li == 0 && pp < nglobal) scores[pp] = s * inverse_root;
        }
    }
    if (has_new && tid < 8) {
        float k8[8];
        unpack8(*reinterpret_cast<const uint4*>(&new_s[0][8 * li]), k8);
        const float s = score_row(q8, k8);
        if (li == 0) scores[nglobal] = s * inverse_root;
    }
    __syncthreads();

    // 4. peak (order-free) and the fast_exp weights
    float m = -INFINITY;
    for (int pp = tid; pp < length; pp += 256) m = fmaxf(m, scores[pp]);
    m = wave_max(m);
    if ((tid & 63) == 0) peak_s[tid >> 6] = m;
    __syncthreads();
    const float peak = fmaxf(fmaxf(peak_s[0], peak_s[1]), fmaxf(peak_s[2], peak_s[3]));
    for (int pp = tid; pp < length; pp += 256) scores[pp] = fast_exp(scores[pp] - peak);
    __syncthreads();

    // 5. weighted values (T3): thread (j, dg) walks positions j, j+16, ... in order
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float total = 0.0f;
    for (int base = 0; base < nglobal; base += 16 * kVChunk) {
        if (base > 0) {
#pragma unroll
            for (int c = 0; c < kVChunk; ++c) {
                const int pp = base + j + 16 * c;
                vr[c] = *reinterpret_cast<const uint2*>(V + (size_t)min(pp, last) * kHeadDim + 4 * dg);
            }
        }
#pragma unroll
        for (int c = 0; c < kVChunk; ++c) {
            const int pp = base + j + 16 * c;
            const bool ok = pp < nglobal;
            const float e = scores[min(pp, last)];
            float v4[4];
            unpack4(vr[c], v4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float t = acc[i] + e * v4[i];
                acc[i] = ok ? t : acc[i];
            }
            const float tt = total + e;
            total = ok ? tt : total;
        }
    }
    if (has_new && j == (nglobal & 15)) {  // the newest position closes its class's sequence
        const float e = scores[nglobal];
        float v4[4];
        unpack4(*reinterpret_cast<const uint2*>(&new_s[1][4 * dg]), v4);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = acc[i] + e * v4[i];
        total = total + e;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) part_s[j][4 * dg + i] = acc[i];
    if (dg == 0) total_s[j] = total;
    __syncthreads();
    if (tid < kHeadDim) {
        float o = 0.0f, t = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            o = o + part_s[k][tid];
            t = t + total_s[k];
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
