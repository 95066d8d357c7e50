// rn_attention.hip — attention over a contiguous fp16 KV cache for gfx950.
//
// Replaces AttentionWeights::attend / attend_heads (crates/model/src/attention.rs:
// 96-213) and kernels::attend_head (crates/kernels/src/attention.rs:251-280) for
// an fp16 cache: score = q.k / sqrt(head_dim), peak-subtracted fast_exp weights,
// weighted values, one multiply by 1/total.
//
// One 256-thread block per (head, query). Latency is the enemy at these sizes
// (a head's cache is 2 x L x 128 bytes), so the first chunk of key rows and of
// value rows (384 positions each) is loaded before the block even reads the
// current position: only then does it read its q/k/v row, apply the rotary and
// append the new key/value, which is served from LDS.
//
// Scores: 4 lanes per key row, 32 bytes (16 dims) each; the block covers 64
// rows per pass. Values: 8 lanes per row, 16 bytes (8 dims) each; thread
// (j, dg) walks positions j, j+32, j+64, ... The float reductions follow the
// fixed trees of the CPU restatement:
//   score (T2): per 4 dims 0 + q0k0 + ... + q3k3; the 16 sub-sums combined by a
//               balanced pairwise tree (two levels inside a lane, then xor 1,
//               xor 2 across the 4 lanes);
//   total and P.V (T3): thirty-two running sums over positions j, j+32, ... in
//               increasing order, then added j = 0..31.
// Scores live in LDS (dynamic, one float per position).
#include "rn_device.hpp"
#include "rn_internal.hpp"

namespace rn {

constexpr int kHeadDim = 64;
constexpr int kClasses = 32;  // T3 position classes (p mod 32)

__device__ __forceinline__ void unpack8(const uint4& raw, float* out) {
    const __half2* h = reinterpret_cast<const __half2*>(&raw);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[2 * i] = __low2float(h[i]);
        out[2 * i + 1] = __high2float(h[i]);
    }
}

// T2 for one key row held as 16 dims per lane (lane li owns dims 16li..16li+15,
// i.e. the four 4-dim sub-sums 4li..4li+3): two tree levels inside the lane,
// the last two across lanes (xor 1, xor 2).
__device__ __forceinline__ float score_row(const float* q16, const uint4& ka, const uint4& kb) {
    float k[16];
    unpack8(ka, k);
    unpack8(kb, k + 8);
    float part[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) s = s + q16[4 * j + i] * k[4 * j + i];
        part[j] = s;
    }
    float s = (part[0] + part[1]) + (part[2] + part[3]);
    s = s + __shfl_xor(s, 1, 4);
    s = s + __shfl_xor(s, 2, 4);
    return s;
}

// KC key passes of 64 rows and VC value positions per thread are issued
// together (64*KC and 32*VC positions). POS_FIRST (decode of many sequences):
// read the position before the cache loads and clamp them to it, instead of
// to the capacity, so that short caches do not fetch the rows of long ones.
template <int MODE, int KC, int VC, bool POS_FIRST>
__global__ __launch_bounds__(256) void attend_kernel(AttendParams p) {
    extern __shared__ float scores[];
    __shared__ float q_s[kHeadDim];
    __shared__ __align__(16) __half new_s[2][kHeadDim];  // decode: the appended key and value
    __shared__ float part_s[kClasses][kHeadDim];
    __shared__ float total_s[kClasses];
    __shared__ float peak_s[4];

    const int tid = threadIdx.x;
    const int r = tid >> 2, li = tid & 3;    // score layout: row slot (64 per pass), 16-dim lane
    const int j = tid >> 3, dg = tid & 7;    // value layout: position class (32), 8-dim lane

    const __half* K;
    const __half* V;
    float* out;
    int nglobal;     // positions read from the cache in global memory
    bool has_new;    // decode: one more position (index nglobal) served from LDS
    int rows;        // rows that exist in this (layer, head) cache: loads clamp to them
    int pos = 0;

    if constexpr (MODE == kAttendDecode) {
        const int h = blockIdx.x, b = blockIdx.y;
        const size_t base = (size_t)b * p.seq_stride + ((size_t)p.layer * p.heads + h) * p.capacity * kHeadDim;
        K = p.kc + base;
        V = p.vc + base;
        out = p.out + (size_t)b * p.d_model + h * kHeadDim;
        rows = p.capacity;
    } else if constexpr (MODE == kAttendPrefill) {
        const int h = blockIdx.x, t = blockIdx.y;
        const size_t base = ((size_t)p.layer * p.heads + h) * p.capacity * kHeadDim;
        K = p.kc + base;
        V = p.vc + base;
        out = p.out + (size_t)t * p.d_model + h * kHeadDim;
        rows = p.capacity;
    } else {
        const int i = blockIdx.x;
        K = p.kc + (size_t)i * p.stride * kHeadDim;
        V = p.vc + (size_t)i * p.stride * kHeadDim;
        out = p.out + (size_t)i * kHeadDim;
        rows = p.stride;
    }

    if constexpr (POS_FIRST) {
        pos = p.pos[(size_t)blockIdx.y * p.pos_stride];
        if (pos < 0 || pos >= p.capacity) {
            if (tid == 0) atomicOr(p.error, 2);
            return;
        }
        rows = pos > 0 ? pos : 1;  // the cached rows; the new one is served from LDS
    }

    // 1. cache loads, issued before anything that depends on the current token
    // or even on the length: rows past the valid ones are clamped into the
    // cache and their results discarded by selects (never by branches, which
    // would split the load stream and force a full wait).
    uint4 kr[KC][2];
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        const __half* row = K + (size_t)min(r + 64 * c, rows - 1) * kHeadDim + 16 * li;
        kr[c][0] = *reinterpret_cast<const uint4*>(row);
        kr[c][1] = *reinterpret_cast<const uint4*>(row + 8);
    }
    uint4 vr[VC];
#pragma unroll
    for (int c = 0; c < VC; ++c)
        vr[c] = *reinterpret_cast<const uint4*>(V + (size_t)min(j + kClasses * c, rows - 1) * kHeadDim + 8 * dg);

    // 2. the length, the query and (decoding) the rotary + fp16 append of the new row
    if constexpr (MODE == kAttendDecode) {
        const int h = blockIdx.x, b = blockIdx.y;
        if constexpr (!POS_FIRST) {
            pos = p.pos[(size_t)b * p.pos_stride];
            if (pos < 0 || pos >= p.capacity) {
                if (tid == 0) atomicOr(p.error, 2);
                return;
            }
        }
        nglobal = pos;
        has_new = true;
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
        nglobal = p.first + blockIdx.y + 1;
        has_new = false;
        if (tid < kHeadDim) q_s[tid] = p.q[(size_t)blockIdx.y * p.d_model + blockIdx.x * kHeadDim + tid];
    } else {
        nglobal = p.lengths[blockIdx.x];
        has_new = false;
        if (nglobal < 1 || nglobal > p.stride) {
            if (tid == 0) atomicOr(p.error, 4);
            return;
        }
        if (tid < kHeadDim) q_s[tid] = p.q[(size_t)blockIdx.x * kHeadDim + tid];
    }
    const int length = nglobal + (has_new ? 1 : 0);
    __syncthreads();

    // 3. scores (T2): one key row per 4-lane group, 64 rows per pass
    const float inverse_root = 1.0f / sqrtf((float)kHeadDim);
    float q16[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) q16[i] = q_s[16 * li + i];
    for (int base = 0; base < nglobal; base += 64 * KC) {
        if (base > 0) {
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                const __half* row = K + (size_t)min(base + r + 64 * c, rows - 1) * kHeadDim + 16 * li;
                kr[c][0] = *reinterpret_cast<const uint4*>(row);
                kr[c][1] = *reinterpret_cast<const uint4*>(row + 8);
            }
        }
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const int pp = base + r + 64 * c;
            const float s = score_row(q16, kr[c][0], kr[c][1]);
            if (li == 0 && pp < nglobal) scores[pp] = s * inverse_root;
        }
    }
    if (has_new && tid < 4) {
        const uint4 ka = *reinterpret_cast<const uint4*>(&new_s[0][16 * li]);
        const uint4 kb = *reinterpret_cast<const uint4*>(&new_s[0][16 * li + 8]);
        const float s = score_row(q16, ka, kb);
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

    // 5. weighted values (T3): thread (j, dg) walks positions j, j+32, ... in order
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    float total = 0.0f;
    const int last = nglobal > 0 ? nglobal - 1 : 0;
    for (int base = 0; base < nglobal; base += kClasses * VC) {
        if (base > 0) {
#pragma unroll
            for (int c = 0; c < VC; ++c)
                vr[c] = *reinterpret_cast<const uint4*>(V + (size_t)min(base + j + kClasses * c, rows - 1) * kHeadDim +
                                                        8 * dg);
        }
#pragma unroll
        for (int c = 0; c < VC; ++c) {
            const int pp = base + j + kClasses * c;
            const bool ok = pp < nglobal;
            const float e = scores[min(pp, last)];
            float v8[8];
            unpack8(vr[c], v8);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float t = acc[i] + e * v8[i];
                acc[i] = ok ? t : acc[i];
            }
            const float tt = total + e;
            total = ok ? tt : total;
        }
    }
    if (has_new && j == (nglobal & (kClasses - 1))) {  // the newest position closes its class
        const float e = scores[nglobal];
        float v8[8];
        unpack8(*reinterpret_cast<const uint4*>(&new_s[1][8 * dg]), v8);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = acc[i] + e * v8[i];
        total = total + e;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) part_s[j][8 * dg + i] = acc[i];
    if (dg == 0) total_s[j] = total;
    __syncthreads();
    if (tid < kHeadDim) {
        float o = 0.0f, t = 0.0f;
#pragma unroll
        for (int k = 0; k < kClasses; ++k) {
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
            if (grid_y == 1)  // one sequence: its loads go out before its position is read
                rn_launch((attend_kernel<kAttendDecode, 6, 12, false>), grid, dim3(256), lds, stream, p);
            else              // many ragged sequences: exact clamps, one pass up to 576 positions
                rn_launch((attend_kernel<kAttendDecode, 9, 18, true>), grid, dim3(256), lds, stream, p);
            break;
        case kAttendPrefill:
            rn_launch((attend_kernel<kAttendPrefill, 4, 8, false>), grid, dim3(256), lds, stream, p);
            break;
        case kAttendRaw:
            rn_launch((attend_kernel<kAttendRaw, 6, 12, false>), grid, dim3(256), lds, stream, p);
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
    rn_launch(rope_append_kernel, dim3(count), dim3(256), 0, stream, qkv, q_out, kc, vc, layer, heads,
                       capacity, d_model, first, rope_cos, rope_sin);
    return hipGetLastError();
}

}  // namespace rn
