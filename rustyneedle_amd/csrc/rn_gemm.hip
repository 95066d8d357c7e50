// rn_gemm.hip — multi-token quantised products on gfx950 i8 MFMA, plus the
// row kernels of batched prefill / multi-sequence decode.
//
// Replaces QuantisedMatrix::multiply_batch / multiply_natural_fused
// (crates/kernels/src/matrix.rs:277-389) and the panel tile
// (crates/kernels/src/panel.rs:136-198) for int8 codes with one fp32 scale per
// 32 columns.
//
// One v_mfma_i32_32x32x32_i8 covers exactly one 32-column group for a 32-token
// x 32-row tile, so every group's int32 accumulators come out of the matrix
// core separately and feed the sequential group epilogue of the reference
// (panel form fmaf(acc, sW*sx, total), or plane form total + (acc*sW)*sx).
// A 256-thread block is 2x2 waves over a 64-token x 64-row output tile; each
// wave streams its 32 token rows and 32 weight rows straight from global
// memory with 128-bit loads (one per lane per group, prefetched one group
// ahead). The finished tile goes through LDS for coalesced stores with the
// fused tail: store, residual add, or silu(gate)*up.
//
// MFMA operand layout (32x32x32 i8): lane l supplies A row l%32 and B column
// l%32, 16 bytes of K from half (l/32); any K permutation inside the
// instruction is the same for A and B, so the group sum is exact regardless.
// Output register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#include "rn_device.hpp"
#include "rn_internal.hpp"

namespace rn {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v4i load16(const int8_t* p, bool ok) {
    if (!ok) return v4i{0, 0, 0, 0};
    const int4 t = *reinterpret_cast<const int4*>(p);
    return v4i{t.x, t.y, t.z, t.w};
}

template <int EPI, int FORM, bool DUMP>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
    __shared__ float tile[64][65];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int G = p.K / kGroup;
    const int m0 = blockIdx.y * 64 + wm * 32;
    int n_base;
    if constexpr (EPI == kGemmSilu)
        n_base = (wn == 0 ? 0 : p.half) + blockIdx.x * 32;
    else
        n_base = blockIdx.x * 64 + wn * 32;
    const int n = n_base + (lane & 31);
    const bool b_ok = n < p.N;
    const int mrow = m0 + (lane & 31);
    const bool a_ok = mrow < p.M;
    const int khalf = (lane >> 5) * 16;
    const int8_t* xa = p.X + (size_t)(a_ok ? mrow : 0) * p.K + khalf;
    const int8_t* wb = p.W + (size_t)(b_ok ? n : 0) * p.K + khalf;
    const float* srow = p.sW + (size_t)(b_ok ? n : 0) * G;

    float sxr[16];
    float total[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int m = m0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        sxr[r] = m < p.M ? p.sx[m] : 0.0f;
        total[r] = 0.0f;
    }

    v4i a = load16(xa, a_ok);
    v4i b = load16(wb, b_ok);
    for (int g = 0; g < G; ++g) {
        v4i an = a, bn = b;
        if (g + 1 < G) {
            an = load16(xa + (g + 1) * kGroup, a_ok);
            bn = load16(wb + (g + 1) * kGroup, b_ok);
        }
        v16i acc = {};
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc, 0, 0, 0);
        const float s = b_ok ? srow[g] : 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            if constexpr (FORM == kPanel)
                total[r] = fmaf((float)acc[r], s * sxr[r], total[r]);  // panel.rs:184-188
            else
                total[r] = total[r] + ((float)acc[r] * s) * sxr[r];    // neon.rs:180
        }
        if constexpr (DUMP) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < p.M && b_ok) p.acc[((size_t)m * p.N + n) * G + g] = acc[r];
            }
        }
        a = an;
        b = bn;
    }

#pragma unroll
    for (int r = 0; r < 16; ++r) tile[wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)][wn * 32 + (lane & 31)] = total[r];
    __syncthreads();

    if constexpr (EPI == kGemmSilu) {
        for (int idx = threadIdx.x; idx < 64 * 32; idx += 256) {
            const int mi = idx >> 5, ii = idx & 31;
            const int m = blockIdx.y * 64 + mi, i = blockIdx.x * 32 + ii;
            if (m < p.M && i < p.half) p.Y[(size_t)m * p.ldy + i] = silu(tile[mi][ii]) * tile[mi][32 + ii];
        }
    } else {
        for (int idx = threadIdx.x; idx < 64 * 64; idx += 256) {
            const int mi = idx >> 6, ni = idx & 63;
            const int m = blockIdx.y * 64 + mi, nn = blockIdx.x * 64 + ni;
            if (m < p.M && nn < p.N) {
                float* dst = p.Y + (size_t)m * p.ldy + nn;
                if constexpr (EPI == kGemmResidual)
                    *dst = *dst + tile[mi][ni];
                else
                    *dst = tile[mi][ni];
            }
        }
    }
}

hipError_t launch_gemm(const GemmParams& p, int epilogue, int form, bool dump, hipStream_t stream) {
    if (p.M <= 0) return hipSuccess;
    if (p.K % kGroup != 0 || p.K <= 0) return hipErrorInvalidValue;
    const int gy = (p.M + 63) / 64;
    int gx;
    if (epilogue == kGemmSilu) {
        if (p.half % 32 != 0 || p.N != 2 * p.half) return hipErrorInvalidValue;
        gx = p.half / 32;
    } else {
        gx = (p.N + 63) / 64;
    }
    const dim3 grid(gx, gy), block(256);
    if (dump) {
        if (epilogue != kGemmStore) return hipErrorInvalidValue;
        if (form == kPanel)
            rn_launch((gemm_kernel<kGemmStore, kPanel, true>), grid, block, 0, stream, p);
        else
            rn_launch((gemm_kernel<kGemmStore, kPlane, true>), grid, block, 0, stream, p);
        return hipGetLastError();
    }
    if (form == kPlane) {
        if (epilogue != kGemmStore) return hipErrorInvalidValue;
        rn_launch((gemm_kernel<kGemmStore, kPlane, false>), grid, block, 0, stream, p);
        return hipGetLastError();
    }
    switch (epilogue) {
        case kGemmStore:
            rn_launch((gemm_kernel<kGemmStore, kPanel, false>), grid, block, 0, stream, p);
            break;
        case kGemmResidual:
            rn_launch((gemm_kernel<kGemmResidual, kPanel, false>), grid, block, 0, stream, p);
            break;
        case kGemmSilu:
            rn_launch((gemm_kernel<kGemmSilu, kPanel, false>), grid, block, 0, stream, p);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- row kernels for multi-token work -------------------------------------------

constexpr int kMaxWidth = 4096;

// Optional zero-centred norm (ops.rs:44-50 with the sum of ops.rs:7-17), then
// the per-row int8 quantisation (ops.rs:112-118). One 64-lane block per row.
// `normed` (nullable) receives the normed row.
__global__ __launch_bounds__(64) void norm_quantise_kernel(const float* x, const float* gain, int n, float eps,
                                                           int8_t* codes, float* scales, float* normed) {
    __shared__ float v[kMaxWidth];
    __shared__ float lanes_s[8];
    const int lane = threadIdx.x;
    const float* row = x + (size_t)blockIdx.x * n;
    for (int i = lane; i < n; i += 64) v[i] = row[i];
    __syncthreads();
    if (gain != nullptr) {
        if (lane < 8) {
            float s = 0.0f;
            for (int c = 0; c < n / 8; ++c) {
                const float t = v[8 * c + lane];
                s = s + t * t;
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
        __syncthreads();
        for (int i = lane; i < n; i += 64) v[i] = ((1.0f + gain[i]) * v[i]) * inverse;
        __syncthreads();
        if (normed != nullptr)
            for (int i = lane; i < n; i += 64) normed[(size_t)blockIdx.x * n + i] = v[i];
    }
    float peak = 0.0f;
    for (int i = lane; i < n; i += 64) peak = fmaxf(peak, fabsf(v[i]));
    peak = wave_max(peak);
    const float scale = int8_scale_from_peak(peak);
    if (codes != nullptr)
        for (int i = lane; i < n; i += 64) codes[(size_t)blockIdx.x * n + i] = (int8_t)quantise_one(v[i], scale);
    if (lane == 0 && scales != nullptr) scales[blockIdx.x] = scale;
}

hipError_t launch_norm_quantise(const float* x, const float* gain, int count, int n, float eps, int8_t* codes,
                                float* scales, float* normed, hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    if (n <= 0 || n > kMaxWidth || n % 8 != 0) return hipErrorInvalidValue;
    rn_launch(norm_quantise_kernel, dim3(count), dim3(64), 0, stream, x, gain, n, eps, codes, scales,
                       normed);
    return hipGetLastError();
}

// Embedding rows (matrix.rs:140-153 for int8 codes) times sqrt(d)
// (session.rs:85-90) for `count` tokens; tokens from `tokens` or, when
// `tokens` is null, from the per-sequence argmax of the previous step.
__global__ __launch_bounds__(256) void embed_rows_kernel(const uint32_t* tokens, const int8_t* E, const float* sE,
                                                         int d, int vocab, float scale, float* X, int32_t* error) {
    uint32_t t = tokens[blockIdx.x];
    if (t >= (uint32_t)vocab) {
        if (threadIdx.x == 0) atomicOr(error, 1);
        t = 0;
    }
    const int G = d / kGroup;
    for (int k = threadIdx.x; k < d; k += blockDim.x)
        X[(size_t)blockIdx.x * d + k] = ((float)E[(size_t)t * d + k] * sE[(size_t)t * G + k / kGroup]) * scale;
}

hipError_t launch_embed_rows(const uint32_t* tokens, int count, const int8_t* E, const float* sE, int d, int vocab,
                             float scale, float* X, int32_t* error, hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    rn_launch(embed_rows_kernel, dim3(count), dim3(256), 0, stream, tokens, E, sE, d, vocab, scale, X, error);
    return hipGetLastError();
}

// generator.rs:257-265 per row: first index of the strict maximum, NaN at
// index 0 wins, other NaNs never do. Writes tokens[row] and ids[row*steps+step].
__global__ __launch_bounds__(256) void argmax_rows_kernel(const float* logits, int n, uint32_t* tokens, uint32_t* ids,
                                                          int steps, int step) {
    __shared__ unsigned long long best_s[4];
    const float* row = logits + (size_t)blockIdx.x * n;
    uint64_t key = 0ull;
    for (int i = threadIdx.x; i < n; i += 256) {
        const uint64_t k = argmax_key(row[i], (uint32_t)i);
        key = k > key ? k : key;
    }
    key = wave_max_u64(key);
    if ((threadIdx.x & 63) == 0) best_s[threadIdx.x >> 6] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t k = best_s[0];
        for (int w = 1; w < 4; ++w) k = best_s[w] > k ? best_s[w] : k;
        const float first = row[0];
        const uint32_t index = (first != first) ? 0u : argmax_index(k);
        tokens[blockIdx.x] = index;
        if (ids != nullptr) ids[(size_t)blockIdx.x * steps + step] = index;
    }
}

hipError_t launch_argmax_rows(const float* logits, int count, int n, uint32_t* tokens, uint32_t* ids, int steps,
                              int step, hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    rn_launch(argmax_rows_kernel, dim3(count), dim3(256), 0, stream, logits, n, tokens, ids, steps, step);
    return hipGetLastError();
}

__global__ void advance_positions_kernel(int32_t* pos, int count, int by) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) pos[i] = pos[i] + by;
}

hipError_t launch_advance_positions(int32_t* pos, int count, int by, hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    rn_launch(advance_positions_kernel, dim3((count + 255) / 256), dim3(256), 0, stream, pos, count, by);
    return hipGetLastError();
}

}  // namespace rn
