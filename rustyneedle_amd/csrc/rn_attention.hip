// rn_attention.hip — attention over a contiguous fp16 KV cache for gfx950.
//
// Replaces AttentionWeights::attend / attend_heads (crates/model/src/attention.rs:
// 96-213) and kernels::attend_head (crates/kernels/src/attention.rs:251-280) for
// an fp16 cache: score = q.k / sqrt(head_dim), peak-subtracted fast_exp weights,
// weighted values, one multiply by 1/total.
//
// One block per (head, query): 256 threads, or 512 for the decode of many
// sequences. Latency is the enemy at these sizes (a head's cache is
// 2 x L x 128 bytes), so the first chunk of key rows and of value rows is
// loaded before the block even reads its q/k/v row, applies the rotary and
// appends the new key/value, which is served from LDS.
//
// Scores: 4 lanes per key row, 32 bytes (16 dims) each; the block covers NT/4
// rows per pass. Values: NT/32 lanes per row (8 or 4 dims each); thread
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

// DPV consecutive fp16 values of one value row: the load type and its floats
template <int DPV> struct ValuePiece;
template <> struct ValuePiece<8> { using T = uint4; };
template <> struct ValuePiece<4> { using T = uint2; };
template <int DPV>
__device__ __forceinline__ void unpack_values(const typename ValuePiece<DPV>::T& raw, float* out) {
    const __half2* h = reinterpret_cast<const __half2*>(&raw);
#pragma unroll
    for (int i = 0; i < DPV / 2; ++i) {
        out[2 * i] = __low2float(h[i]);
        out[2 * i + 1] = __high2float(h[i]);
    }
}

// T2 for one key row held as 16 dims per lane (lane li owns dims 16li..16li+15,
// i.e. the four 4-dim sub-sums 4li..4li+3): two tree levels inside the lane,
// the last two across lanes (xor 1, xor 2; the four lanes of a row are one
// DPP quad).
__device__ __forceinline__ float score_row(const float* q16, const uint4& ka, const uint4& kb) {
    // dims 2w and 2w + 1 are the low and high halves of word w
    const uint32_t w[8] = {ka.x, ka.y, ka.z, ka.w, kb.x, kb.y, kb.z, kb.w};
    float part[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float s = 0.0f;
        s = s + mul_f16<false>(q16[4 * j], w[2 * j]);
        s = s + mul_f16<true>(q16[4 * j + 1], w[2 * j]);
        s = s + mul_f16<false>(q16[4 * j + 2], w[2 * j + 1]);
        s = s + mul_f16<true>(q16[4 * j + 3], w[2 * j + 1]);
        part[j] = s;
    }
    float s = (part[0] + part[1]) + (part[2] + part[3]);
    s = s + __int_as_float(dpp_move<0xb1>(__float_as_int(s)));  // lane ^ 1
    s = s + __int_as_float(dpp_move<0x4e>(__float_as_int(s)));  // lane ^ 2
    return s;
}

// KC key passes of NT/4 rows and VC value positions per thread are issued
// together (NT/4*KC and 32*VC positions); NT threads, 4 lanes per key row and
// NT/32 lanes per position class. POS_FIRST (decode of many sequences): read
// the position before the cache loads and clamp them to it, instead of to the
// capacity, so that short caches do not fetch the rows of long ones. Passes and
// value slots past the length are skipped per wave (they add nothing).
template <int MODE, int KC, int VC, bool POS_FIRST, int NT = 256>
// (512-thread blocks are held to 128 VGPRs, so that two blocks share a CU)
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(NT >= 512 ? 4 : 1))) void attend_kernel(
    AttendParams p) {
    constexpr int KROWS = NT / 4;         // key rows per pass (4 lanes per row)
    constexpr int TPC = NT / kClasses;    // value threads per position class
    constexpr int DPV = kHeadDim / TPC;   // value dims per thread
    using VPiece = typename ValuePiece<DPV>::T;
    extern __shared__ float scores[];
    __shared__ float q_s[kHeadDim];
    __shared__ __align__(16) __half new_s[2][kHeadDim];  // decode: the appended key and value
    __shared__ float part_s[kClasses][kHeadDim];
    __shared__ float total_s[kClasses];
    __shared__ float peak_s[NT / 64];

    const int tid = threadIdx.x, wave = tid >> 6;
    const int r = tid >> 2, li = tid & 3;     // score layout: row slot (KROWS per pass), 16-dim lane
    const int j = tid / TPC, dg = tid % TPC;  // value layout: position class (32), DPV-dim lane

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

    // the new q/k/v row and its rotary factors (decoding many sequences): requested
    // before the cache rows, so that the query is ready when the keys arrive
    float nq[2] = {0.0f, 0.0f}, nk[2] = {0.0f, 0.0f}, nv[2] = {0.0f, 0.0f}, rc = 0.0f, rsn = 0.0f;
    if constexpr (MODE == kAttendDecode && POS_FIRST) {
        if (tid < kHeadDim / 2) {
            const float* row = p.qkv + (size_t)blockIdx.y * 3 * p.d_model + blockIdx.x * kHeadDim + tid;
            nq[0] = row[0];
            nq[1] = row[kHeadDim / 2];
            nk[0] = row[p.d_model];
            nk[1] = row[p.d_model + kHeadDim / 2];
            nv[0] = row[2 * p.d_model];
            nv[1] = row[2 * p.d_model + kHeadDim / 2];
        }
    }
    if constexpr (POS_FIRST) {
        pos = p.pos[(size_t)blockIdx.y * p.pos_stride];
        if (pos < 0 || pos >= p.capacity) {
            if (tid == 0) atomicOr(p.error, 2);
            return;
        }
        rows = pos > 0 ? pos : 1;  // the cached rows; the new one is served from LDS
        if constexpr (MODE == kAttendDecode) {
            if (tid < kHeadDim / 2) {
                rc = p.rope_cos[(size_t)pos * (kHeadDim / 2) + tid];
                rsn = p.rope_sin[(size_t)pos * (kHeadDim / 2) + tid];
            }
        }
    }

    // 1. cache loads, issued before anything that depends on the current token
    // or even on the length: rows past the valid ones are clamped into the
    // cache and their results discarded by selects (never by branches, which
    // would split the load stream and force a full wait).
    uint4 kr[KC][2];
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        const __half* row = K + (size_t)min(r + KROWS * c, rows - 1) * kHeadDim + 16 * li;
        kr[c][0] = *reinterpret_cast<const uint4*>(row);
        kr[c][1] = *reinterpret_cast<const uint4*>(row + 8);
    }
    VPiece vr[VC];
#pragma unroll
    for (int c = 0; c < VC; ++c)
        vr[c] = *reinterpret_cast<const VPiece*>(V + (size_t)min(j + kClasses * c, rows - 1) * kHeadDim + DPV * dg);

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
            float c, s, qa, qb, ka, kb, va, vb;
            if constexpr (POS_FIRST) {  // requested before the cache rows
                c = rc, s = rsn, qa = nq[0], qb = nq[1], ka = nk[0], kb = nk[1], va = nv[0], vb = nv[1];
            } else {
                c = p.rope_cos[(size_t)pos * half + i];
                s = p.rope_sin[(size_t)pos * half + i];
                qa = row[h * kHeadDim + i], qb = row[h * kHeadDim + i + half];
                ka = row[p.d_model + h * kHeadDim + i], kb = row[p.d_model + h * kHeadDim + i + half];
                va = row[2 * p.d_model + h * kHeadDim + i], vb = row[2 * p.d_model + h * kHeadDim + i + half];
            }
            q_s[i] = qa * c - qb * s;
            q_s[i + half] = qb * c + qa * s;
            const __half k0 = __float2half_rn(ka * c - kb * s), k1 = __float2half_rn(kb * c + ka * s);
            const __half v0 = __float2half_rn(va);
            const __half v1 = __float2half_rn(vb);
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
    for (int base = 0; base < nglobal; base += KROWS * KC) {
        if (base > 0) {
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                const __half* row = K + (size_t)min(base + r + KROWS * c, rows - 1) * kHeadDim + 16 * li;
                kr[c][0] = *reinterpret_cast<const uint4*>(row);
                kr[c][1] = *reinterpret_cast<const uint4*>(row + 8);
            }
        }
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const int pp = base + r + KROWS * c;
            if (base + KROWS * c + 16 * wave < nglobal) {  // wave-uniform: the wave's rows hold live positions
                const float s = score_row(q16, kr[c][0], kr[c][1]);
                if (li == 0 && pp < nglobal) scores[pp] = s * inverse_root;
            }
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
    for (int pp = tid; pp < length; pp += NT) m = fmaxf(m, scores[pp]);
    m = wave_max(m);
    if ((tid & 63) == 0) peak_s[wave] = m;
    __syncthreads();
    float peak = peak_s[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) peak = fmaxf(peak, peak_s[w]);
    for (int pp = tid; pp < length; pp += NT) scores[pp] = fast_exp(scores[pp] - peak);
    __syncthreads();

    // 5. weighted values (T3): thread (j, dg) walks positions j, j+32, ... in order
    float acc[DPV];
#pragma unroll
    for (int i = 0; i < DPV; ++i) acc[i] = 0.0f;
    float total = 0.0f;
    const int last = nglobal > 0 ? nglobal - 1 : 0;
    for (int base = 0; base < nglobal; base += kClasses * VC) {
        if (base > 0) {
#pragma unroll
            for (int c = 0; c < VC; ++c)
                vr[c] = *reinterpret_cast<const VPiece*>(V + (size_t)min(base + j + kClasses * c, rows - 1) * kHeadDim +
                                                         DPV * dg);
        }
        // the weights of all slots are read from LDS before the slot tests (a
        // read inside each test would be waited for before the next one)
        float ew[VC];
#pragma unroll
        for (int c = 0; c < VC; ++c) ew[c] = scores[min(base + j + kClasses * c, last)];
#pragma unroll
        for (int c = 0; c < VC; ++c) {
            const int pp = base + j + kClasses * c;
            // wave-uniform: the wave's classes hold no live position in this slot
            if (base + kClasses * c + (64 / TPC) * wave >= nglobal) continue;
            const bool ok = pp < nglobal;
            const float e = ew[c];
            const uint32_t* vw = reinterpret_cast<const uint32_t*>(&vr[c]);
#pragma unroll
            for (int i = 0; i < DPV; ++i) {
                const float t = acc[i] + ((i & 1) ? mul_f16<true>(e, vw[i / 2]) : mul_f16<false>(e, vw[i / 2]));
                acc[i] = ok ? t : acc[i];
            }
            const float tt = total + e;
            total = ok ? tt : total;
        }
    }
    if (has_new && j == (nglobal & (kClasses - 1))) {  // the newest position closes its class
        const float e = scores[nglobal];
        float vv[DPV];
        unpack_values<DPV>(*reinterpret_cast<const VPiece*>(&new_s[1][DPV * dg]), vv);
#pragma unroll
        for (int i = 0; i < DPV; ++i) acc[i] = acc[i] + e * vv[i];
        total = total + e;
    }
#pragma unroll
    for (int i = 0; i < DPV; ++i) part_s[j][DPV * dg + i] = acc[i];
    if (dg == 0) total_s[j] = total;
    __syncthreads();
    if (tid < kHeadDim) {
        float o = 0.0f, t = 0.0f;
#pragma unroll
        for (int k = 0; k < kClasses; ++k) {
            o = o + part_s[k][tid];
            t = t + total_s[k];
        }
        const float inverse = reciprocal(t);
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
                rn_launch((attend_kernel<kAttendDecode, 5, 18, true, 512>), grid, dim3(512), lds, stream, p);
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

// Causal prefill attention over query tiles: one 256-thread block per (head,
// QT consecutive queries), so each key and value row is read from L2 once per
// tile instead of once per query. Rows go to LDS in chunks of 256 positions
// (global_load_lds: no registers); the scores of the QT queries live in LDS
// [QT][length]. The float order is the per-query kernel's: scores in tree T2
// (4 lanes per key row, the row's 16 dims per lane reused for all QT
// queries), peak, fast_exp weights, then the value sums in tree T3 (thread
// (class j, 8 dims) walks positions j, j + 32, ... in order for every query),
// classes added 0..31, one multiply by 1/total.
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void global_void;

constexpr int kTileRows = 256;  // positions per staged chunk

template <int QT>
__global__ __launch_bounds__(256) void attend_prefill_tile_kernel(AttendParams p, int count) {
    constexpr int NT = 256;
    extern __shared__ float scores[];  // [QT][max length]
    __shared__ __align__(16) __half k_s[kTileRows * kHeadDim];  // a chunk of key rows
    __shared__ __align__(16) __half v_s[kTileRows * kHeadDim];  // a chunk of value rows
    __shared__ float q_s[QT][kHeadDim];
    __shared__ float total_s[QT][kClasses];
    float(*part_s)[kClasses][kHeadDim] = reinterpret_cast<float(*)[kClasses][kHeadDim]>(k_s);
    static_assert(QT * kClasses * kHeadDim * 4 <= kTileRows * kHeadDim * 2, "class sums fit in the key buffer");

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // the last tiles attend the most positions: they go first
    const int h = blockIdx.x, t0 = (gridDim.y - 1 - blockIdx.y) * QT;
    const int stride = p.first + count;  // scores row pitch
    const size_t base = ((size_t)p.layer * p.heads + h) * p.capacity * kHeadDim;
    const __half* K = p.kc + base;
    const __half* V = p.vc + base;
    int len[QT];  // positions each query attends (0: a query past the end)
#pragma unroll
    for (int q = 0; q < QT; ++q) len[q] = t0 + q < count ? p.first + t0 + q + 1 : 0;
    const int L = p.first + min(t0 + QT, count);  // rows the tile needs (t0 < count)

    // a chunk of rows [c0, c0 + 256) of K or V into dst; rows past L repeat row L - 1
    auto stage = [&](const __half* src, __half* dst, int c0) {
#pragma unroll
        for (int i = 0; i < kTileRows * 8 / NT; ++i) {
            const int piece = NT * i + 64 * wave + lane, row = min(c0 + piece / 8, L - 1);
            __builtin_amdgcn_global_load_lds((global_void*)(src + (size_t)row * kHeadDim + 8 * (piece % 8)),
                                             (lds_void*)(dst + 8 * (NT * i + 64 * wave)), 16, 0, 0);
        }
    };
    // the first chunks of keys and values are requested together
    stage(K, k_s, 0);
    stage(V, v_s, 0);
    if (tid < QT * kHeadDim) {
        const int q = tid / kHeadDim, d = tid % kHeadDim;
        q_s[q][d] = p.q[(size_t)min(t0 + q, count - 1) * p.d_model + h * kHeadDim + d];
    }

    // 1. scores (T2): key row r of a pass in lanes 4 r .. 4 r + 3, 16 dims each
    const int r = tid >> 2, li = tid & 3;
    const float inverse_root = 1.0f / sqrtf((float)kHeadDim);
    float qr[QT][16];  // this lane's 16 query dims of every query
    for (int c0 = 0; c0 < L; c0 += kTileRows) {
        if (c0 > 0) {
            __syncthreads();  // the previous chunk is consumed
            stage(K, k_s, c0);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (c0 == 0) {
#pragma unroll
            for (int q = 0; q < QT; ++q)
#pragma unroll
                for (int i = 0; i < 16; ++i) qr[q][i] = q_s[q][16 * li + i];
        }
        for (int pass = 0; pass < kTileRows && c0 + pass < L; pass += NT / 4) {
            const int pp = c0 + pass + r;
            const uint4* kr = reinterpret_cast<const uint4*>(k_s + (pass + r) * kHeadDim + 16 * li);
            const uint4 ka = kr[0], kb = kr[1];
#pragma unroll
            for (int q = 0; q < QT; ++q) {
                // the fp16 keys multiply in place (v_fma_mix_f32: the exact product rounded once)
                const float sc = score_row(qr[q], ka, kb);
                if (li == 0 && pp < len[q]) scores[q * stride + pp] = sc * inverse_root;
            }
        }
    }
    __syncthreads();

    // 2. peak (order-free) and the fast_exp weights: wave q serves query q
    for (int q = wave; q < QT; q += NT / 64) {
        const int n = len[q];
        float m = -INFINITY;
        for (int pp = lane; pp < n; pp += 64) m = fmaxf(m, scores[q * stride + pp]);
        m = wave_max(m);
        for (int pp = lane; pp < n; pp += 64) scores[q * stride + pp] = fast_exp(scores[q * stride + pp] - m);
    }

    // 3. weighted values (T3): thread (j, dg) walks positions j, j + 32, ... for every query
    const int j = tid >> 3, dg = tid & 7;
    float acc[QT][8];
    float total[QT];
#pragma unroll
    for (int q = 0; q < QT; ++q) {
        total[q] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[q][i] = 0.0f;
    }
    for (int c0 = 0; c0 < L; c0 += kTileRows) {
        __syncthreads();  // weights written; the previous chunk is consumed
        if (c0 > 0) {
            stage(V, v_s, c0);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
        // positions every query of the tile attends, then the tile's last QT - 1
        const int all = min(c0 + kTileRows, len[0]), end = min(c0 + kTileRows, L);
        int pp = c0 + j;
        // e times the fp16 value by v_fma_mix_f32 (the exact product rounded once)
        auto weigh = [&](float (&a)[8], float e, const uint4& raw) {
            const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
            for (int i = 0; i < 8; ++i)
                a[i] = a[i] + ((i & 1) ? mul_f16<true>(e, w[i / 2]) : mul_f16<false>(e, w[i / 2]));
        };
        for (; pp < all; pp += kClasses) {
            const uint4 raw = *reinterpret_cast<const uint4*>(v_s + (pp - c0) * kHeadDim + 8 * dg);
#pragma unroll
            for (int q = 0; q < QT; ++q) {
                const float e = scores[q * stride + pp];
                weigh(acc[q], e, raw);
                total[q] = total[q] + e;
            }
        }
        for (; pp < end; pp += kClasses) {
            const uint4 raw = *reinterpret_cast<const uint4*>(v_s + (pp - c0) * kHeadDim + 8 * dg);
#pragma unroll
            for (int q = 0; q < QT; ++q) {
                if (pp < len[q]) {
                    const float e = scores[q * stride + pp];
                    weigh(acc[q], e, raw);
                    total[q] = total[q] + e;
                }
            }
        }
    }
    // the key buffer becomes the class sums (its last readers passed the barrier above)
#pragma unroll
    for (int q = 0; q < QT; ++q) {
#pragma unroll
        for (int i = 0; i < 8; ++i) part_s[q][j][8 * dg + i] = acc[q][i];
        if (dg == 0) total_s[q][j] = total[q];
    }
    __syncthreads();
    if (tid < QT * kHeadDim) {
        const int q = tid / kHeadDim, d = tid % kHeadDim;
        if (t0 + q < count) {
            float o = 0.0f, t = 0.0f;
#pragma unroll
            for (int k = 0; k < kClasses; ++k) {
                o = o + part_s[q][k][d];
                t = t + total_s[q][k];
            }
            const float inverse = reciprocal(t);
            p.out[(size_t)(t0 + q) * p.d_model + h * kHeadDim + d] = o * inverse;
        }
    }
}

// The tiled kernel holds the scores of QT queries over the whole length in LDS;
// longer contexts take the per-query kernel.
constexpr int kPrefillTileQueries = 4;
constexpr int kPrefillTileMaxLength = 6144;

hipError_t launch_attend_prefill(const AttendParams& p, int heads, int count, hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    const int length = p.first + count;
    if (length > kPrefillTileMaxLength) return launch_attend(p, kAttendPrefill, heads, count, length, stream);
    const size_t lds = sizeof(float) * (size_t)kPrefillTileQueries * length;
    const dim3 grid(heads, (count + kPrefillTileQueries - 1) / kPrefillTileQueries);
    rn_launch(attend_prefill_tile_kernel<kPrefillTileQueries>, grid, dim3(256), lds, stream, p, count);
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

// Batch-1 decode: the norm + q/k/v product of one head, its rotary and fp16
// append, and its attention, in one 512-thread block per head
// (session.rs:94-120 with model/src/attention.rs:96-154 for one token).
//
// A head needs only its own 192 rows of the fused q/k/v matrix (q, k and v rows
// 64h..64h+63), so the product splits by head with no exchange between blocks.
// The kernel is a chain of dependent steps, so it is laid out to keep global
// loads and barriers off that chain:
//   1. every load is requested at the start: wave 0 the input row (or the
//      embedding row of the token times sqrt(d), session.rs:85-90) and the
//      norm gains; waves 1-6 the head's weight rows and scales; wave 7 the
//      position (one scalar load) and then the rotary angles of that
//      position, for the block through LDS; every wave its share of the first
//      KC x 128 key rows and 32 x VC value rows (clamped to the capacity, so
//      that they need not wait for the position);
//   2. wave 0: zero-centred RMSNorm (eight-lane sum of ops.rs:7-17) and int8
//      codes (ops.rs:103-118) into LDS (barrier 1);
//   3. waves 1-6, 32 rows each, two lanes a row: each lane owns half a row's
//      codes, so its group sums never leave the lane; the panel epilogue
//      fmaf(acc, sW * sx, total) runs in group order over the first half's
//      groups in the even lane and continues in the odd lane (panel.rs:184-188);
//      a wave holds rows i and i + 32 of its section in lanes l and l ^ 32, so
//      the rotate-half rotary (ops.rs:131-141) is a lane swap; q goes to LDS,
//      k and v to LDS and to the cache as fp16 (barrier 2);
//   4. scores (tree T2 of score_row) into LDS with each thread's running peak,
//      the block peak through one barrier (barrier 3), the fast_exp weights
//      (barrier 4), then the value sums in tree T3 (32 position classes, 4 dims
//      per thread, barrier 5) and the class combine with one multiply by
//      1/total.
// The block shares data through LDS only, so its barriers wait for LDS
// operations and not for global loads or stores (the new cache rows it stores
// are read from LDS). The float results are identical to the separate
// product + attend_kernel path.
template <int K, int PRO, int KC, int VC>
__global__ __launch_bounds__(512) void qkv_attend_kernel(QkvAttendParams p) {
    constexpr int NT = 512;
    constexpr int G = K / kGroup;            // weight scales per row
    constexpr int CPR = K / 16;              // 16-code chunks per row
    constexpr int HC = CPR / 2;              // chunks per lane: half a row
    constexpr int HG = G / 2;                // groups per lane
    constexpr int E = K / 64;                // prologue values per lane of wave 0
    constexpr int KROWS = NT / 4;            // key rows per pass
    static_assert(E % 2 == 0 && HG % 2 == 0 && HC == 2 * HG, "whole float pairs, scale pairs, two chunks a group");
    extern __shared__ float scores[];
    __shared__ __align__(16) int8_t xq_s[K];
    __shared__ __align__(16) float sq_s[K];
    __shared__ __align__(16) int acc_s[6 * 32 * CPR];  // chunk sums, 32 rows a product wave
    __shared__ float q_s[kHeadDim];
    __shared__ __align__(16) __half new_s[2][kHeadDim];
    __shared__ __align__(16) float part_s[kClasses][kHeadDim];
    __shared__ float total_s[kClasses];
    __shared__ float peak_s[NT / 64];
    __shared__ float sx_s;
    __shared__ int pos_s;
    __shared__ float rope_s[2][kHeadDim / 2];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = blockIdx.x;
    const int r = tid >> 2, li = tid & 3;     // score layout: key row slot, 16-dim quarter
    const int j = tid >> 4, dq = tid & 15;    // value layout: position class, dims 4dq..4dq+3
    const size_t head_base = (size_t)h * p.capacity * kHeadDim;
    const __half* Kc = p.kc + head_base;
    const __half* Vc = p.vc + head_base;
    // product layout (waves 1-6): section q / k / v, the lane pair of row
    // slot lr, half hh of the row; slots lr and lr ^ 16 hold dims i and i + 32
    const int section = (wave - 1) >> 1, sub = (wave - 1) & 1, lr = lane >> 1, hh = lane & 1;
    auto dim_of = [&](int slot) { return (slot & 15) + 16 * sub + 32 * (slot >> 4); };
    auto slot_row = [&](int slot) { return (size_t)section * K + (size_t)h * kHeadDim + dim_of(slot); };
    const int dim = dim_of(lr);
    const int rot = (lr & 15) + 16 * sub;     // rotary pair index of this row
    const bool rows_wave = wave >= 1 && wave <= 6;
    // The first pass of key and value rows does not wait for the position: a
    // load that needed it would start only when the position's own load came
    // back. The rows are clamped to the capacity instead; rows past the cached
    // ones are read but never used. Each kind of wave issues them in its own
    // branch: a distinct asm statement per branch (after the loads, and the
    // zero `salt` before them) keeps the compiler from merging the copies below
    // the branches, behind the product waves' wait for the position.
    const int top = p.capacity - 1;
    uint4 kr[KC][2];
    uint2 vr[VC];
    auto request_cache = [&](int salt) {
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const __half* row = Kc + (size_t)min(r + KROWS * c, top) * kHeadDim + 16 * li + salt;
            kr[c][0] = *reinterpret_cast<const uint4*>(row);
            kr[c][1] = *reinterpret_cast<const uint4*>(row + 8);
        }
#pragma unroll
        for (int c = 0; c < VC; ++c)
            vr[c] = *reinterpret_cast<const uint2*>(Vc + (size_t)min(j + kClasses * c, top) * kHeadDim + 4 * dq +
                                                    salt);
    };
    int salt;

    // 1. requests: the prologue input first (wave 0), the weights and scales
    // (waves 1-6), the position and the rotary angles (wave 7), the cache rows
    float v[E], gv[E];
    int4 w[HC];
    float sv[HG];
    if (wave == 0) {
        if constexpr (PRO == kEmbedNorm || PRO == kEmbedArgmax) {
            uint32_t token;
            if constexpr (PRO == kEmbedArgmax) {
                // the previous step's greedy choice (generator.rs:257-265): the
                // largest of the logits kernel's block keys (the lowest index
                // among equal values); a NaN at index 0 is never displaced
                // (the lane's sixteen keys of a round of 1024 requested before
                // any compare, from clamped indices: a repeated key does not
                // change the maximum; a loop of single loads waits for each)
                uint64_t key = 0ull;
                for (int base = 0; base < p.nkeys; base += 1024) {
                    uint64_t kk[16];
#pragma unroll
                    for (int i = 0; i < 16; ++i) kk[i] = p.keys[min(base + lane + 64 * i, p.nkeys - 1)];
#pragma unroll
                    for (int i = 0; i < 16; ++i) key = kk[i] > key ? kk[i] : key;
                }
                key = wave_max_u64(key);
                const float first = p.logits[0];
                token = (first != first) ? 0u : argmax_index(key);
                if (h == 0 && lane == 0) {
                    p.state->token = token;
                    const uint32_t step = p.state->step;
                    if (step > 0 && step - 1 < p.state->ids_capacity) p.ids[step - 1] = token;
                }
            } else {
                token = p.state->token;
            }
            if (token >= (uint32_t)p.vocab) {
                if (lane == 0 && h == 0) atomicOr(&p.state->error, 1);
                token = 0;
            }
            const int8_t* er = p.embW + (size_t)token * K + lane * E;
#pragma unroll
            for (int e = 0; e < E; ++e)
                v[e] = ((float)er[e] * p.embS[(size_t)token * G + (lane * E + e) / kGroup]) * p.embed_scale;
            if (h == 0)
#pragma unroll
                for (int e = 0; e < E; ++e) p.x_out[lane * E + e] = v[e];
        } else {
            load_floats<E>(p.x + lane * E, v);
        }
        load_floats<E>(p.gain + lane * E, gv);
        asm volatile("v_mov_b32 %0, 0 ; salt: prologue wave" : "=v"(salt));
        request_cache(salt);
        asm volatile("; requests issued: prologue wave" ::: "memory");
    } else if (rows_wave) {
        // load c covers chunk 64 c + lane of the wave's 32 rows taken slot by
        // slot: consecutive lanes read consecutive 16-byte chunks of a row
#pragma unroll
        for (int c = 0; c < HC; ++c) {
            const int chunk = 64 * c + lane, slot = chunk / CPR;
            w[c] = *reinterpret_cast<const int4*>(p.W + slot_row(slot) * K + (chunk % CPR) * 16);
        }
        load_floats<HG>(p.sW + slot_row(lr) * G + hh * HG, sv);
        asm volatile("v_mov_b32 %0, 0 ; salt: product wave" : "=v"(salt));
        request_cache(salt);
        asm volatile("; requests issued: product wave" ::: "memory");
    } else {
        // wave 7: the position (its wait is this wave's only work before the
        // first barrier) and the rotary angles of the product waves' rows,
        // both through LDS; then its cache rows
        const int pos_in = p.state->pos;
        const int pr = (pos_in < 0 || pos_in >= p.capacity) ? 0 : pos_in;
        const int half = lane & (kHeadDim / 2 - 1);
        const float angle_cos = p.rope_cos[(size_t)pr * (kHeadDim / 2) + half];
        const float angle_sin = p.rope_sin[(size_t)pr * (kHeadDim / 2) + half];
        asm volatile("v_mov_b32 %0, 0 ; salt: attention wave" : "=v"(salt));
        request_cache(salt);
        asm volatile("; requests issued: attention wave" ::: "memory");
        if (lane < kHeadDim / 2) {
            rope_s[0][lane] = angle_cos;
            rope_s[1][lane] = angle_sin;
        }
        if (lane == 0) pos_s = pos_in;
    }

    // 2. wave 0: the norm and the int8 codes (DS operations of a wave complete
    // in order, so the squares need only a wave barrier)
    if (wave == 0) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int idx = lane * E + e;
            sq_s[(idx % 8) * (K / 8) + idx / 8] = v[e] * v[e];
        }
        // the gained values m = (1 + g) x and their peak while the squares'
        // LDS writes complete: the normed value is fl(m * inverse) with
        // inverse > 0 and rounding is monotone, so the normed peak is
        // fl(peak(|m|) * inverse)
        float peak = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            v[e] = (1.0f + gv[e]) * v[e];
            peak = fmaxf(peak, fabsf(v[e]));
        }
        peak = wave_max_nonneg(peak);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float s = 0.0f;
        if (lane < 8) {
            const float4* run = reinterpret_cast<const float4*>(sq_s + lane * (K / 8));
            float4 t[K / 32];
#pragma unroll
            for (int c = 0; c < K / 32; ++c) t[c] = run[c];
#pragma unroll
            for (int c = 0; c < K / 32; ++c) {
                s = s + t[c].x;
                s = s + t[c].y;
                s = s + t[c].z;
                s = s + t[c].w;
            }
        }
        float total = sum_lanes_0_to_7(s);
        total = total + 0.0f;  // the (empty) tail of ops.rs:15-16
        const float inverse = reciprocal(sqrtf(total / (float)K + p.eps));
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = v[e] * inverse;
        const float sx = int8_scale_from_peak(peak * inverse);
        float y[E];
        quotients<E>(v, sx, y);
#pragma unroll
        for (int e = 0; e < E; ++e) xq_s[lane * E + e] = (int8_t)code_of_quotient(y[e]);
        if (lane == 0) sx_s = sx;
    }
    lds_barrier();
    // a position outside the cache is flagged; the block then runs on position 0
    // and stores nothing (uniform over the block)
    const int pos_in = pos_s;
    const bool bad_pos = pos_in < 0 || pos_in >= p.capacity;
    if (bad_pos && tid == 0) atomicOr(&p.state->error, 2);
    const int pos = bad_pos ? 0 : pos_in;
    const int last_row = pos > 0 ? pos - 1 : 0;  // the last cached row (later passes clamp to it)

    // 3. waves 1-6: a row's exact group sums inside its lane pair, the epilogue
    // chain over the even lane's groups continued by the odd lane, the rotary
    // by lane swap, and the stores of q, k and v
    if (rows_wave) {
        // exact int32 sums of 16-code chunks, through this wave's own LDS rows
        // (DS operations of a wave complete in order) to the lane pair of each
        // row, which adds a group's two chunks
        int* wacc = acc_s + (wave - 1) * 32 * CPR;
#pragma unroll
        for (int c = 0; c < HC; ++c) {
            const int chunk = 64 * c + lane;
            wacc[chunk] = dot16(w[c], *reinterpret_cast<const int4*>(xq_s + (chunk % CPR) * 16), 0);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        int acc[HG];
#pragma unroll
        for (int g = 0; g < HG; g += 2) {
            const int4 a4 = *reinterpret_cast<const int4*>(wacc + lr * CPR + hh * HC + 2 * g);
            acc[g] = a4.x + a4.y;
            acc[g + 1] = a4.z + a4.w;
        }
        const float sx = sx_s;
        float scale[HG];
#pragma unroll
        for (int g = 0; g < HG; ++g) scale[g] = sv[g] * sx;
        float first = 0.0f;  // groups 0..HG-1 (meaningful in even lanes)
#pragma unroll
        for (int g = 0; g < HG; ++g) first = fmaf((float)acc[g], scale[g], first);
        float total = lane_xor<1>(first);  // odd lanes continue from the even lane's total
#pragma unroll
        for (int g = 0; g < HG; ++g) total = fmaf((float)acc[g], scale[g], total);
        // lane exchanges run in every lane (a DPP source lane that is off would
        // give the lane its own value), then the selects
        const float from_odd = lane_xor<1>(total);
        const float value = hh ? total : from_odd;  // the row in both lanes of its pair
        const float other = lane_xor<32>(value);    // dim i + 32 for dim i, and back
        if (hh == 0) {
            if (section == 2) {
                const __half vh = __float2half_rn(value);
                new_s[1][dim] = vh;
                if (!bad_pos) const_cast<__half*>(Vc)[(size_t)pos * kHeadDim + dim] = vh;
            } else {
                // rotate-half: (a, b) = (dim i, dim i + 32) -> (a c - b s, b c + a s)
                const float rc = rope_s[0][rot], rs = rope_s[1][rot];
                const float rotated = lr < 16 ? value * rc - other * rs : value * rc + other * rs;
                if (section == 0) {
                    q_s[dim] = rotated;
                } else {
                    const __half kh = __float2half_rn(rotated);
                    new_s[0][dim] = kh;
                    if (!bad_pos) const_cast<__half*>(Kc)[(size_t)pos * kHeadDim + dim] = kh;
                }
            }
        }
    }
    lds_barrier();

    // 4. scores (T2), KROWS key rows per pass, and each thread's peak
    const int nglobal = pos, length = pos + 1;
    const float inverse_root = 1.0f / sqrtf((float)kHeadDim);
    float q16[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) q16[i] = q_s[16 * li + i];
    float m = -INFINITY;
    for (int base = 0; base < nglobal; base += KROWS * KC) {
        if (base > 0) {
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                const __half* row = Kc + (size_t)min(base + r + KROWS * c, last_row) * kHeadDim + 16 * li;
                kr[c][0] = *reinterpret_cast<const uint4*>(row);
                kr[c][1] = *reinterpret_cast<const uint4*>(row + 8);
            }
        }
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const int pp = base + r + KROWS * c;
            if (base + KROWS * c + 16 * wave < nglobal) {  // wave-uniform: the pass holds live rows
                const float s = score_row(q16, kr[c][0], kr[c][1]) * inverse_root;
                if (pp < nglobal) {
                    m = fmaxf(m, s);
                    if (li == 0) scores[pp] = s;
                }
            }
        }
    }
    if (tid >= NT - 4) {  // the last wave: it holds the highest rows of every pass
        const uint4 ka = *reinterpret_cast<const uint4*>(&new_s[0][16 * li]);
        const uint4 kb = *reinterpret_cast<const uint4*>(&new_s[0][16 * li + 8]);
        const float s = score_row(q16, ka, kb) * inverse_root;
        m = fmaxf(m, s);
        if (li == 0) scores[nglobal] = s;
    }
    m = wave_max(m);
    if (lane == 0) peak_s[wave] = m;
    lds_barrier();

    // 5. the fast_exp weights (the peak is order-free)
    float peak = peak_s[0];
#pragma unroll
    for (int w8 = 1; w8 < NT / 64; ++w8) peak = fmaxf(peak, peak_s[w8]);
    for (int pp = tid; pp < length; pp += NT) scores[pp] = fast_exp(scores[pp] - peak);
    lds_barrier();

    // 6. weighted values (T3): thread (j, dq) walks positions j, j+32, ... in order
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float total = 0.0f;
    const int last = nglobal > 0 ? nglobal - 1 : 0;
    for (int base = 0; base < nglobal; base += kClasses * VC) {
        if (base > 0) {
#pragma unroll
            for (int c = 0; c < VC; ++c)
                vr[c] = *reinterpret_cast<const uint2*>(Vc + (size_t)min(base + j + kClasses * c, last_row) *
                                                        kHeadDim + 4 * dq);
        }
        // slots below `whole` hold a live position in every class; slot
        // `whole` (if any) in some; later slots in none (uniform tests). The
        // weights are read from LDS before the tests, all at once.
        const int whole = (nglobal - base) >> 5;
        float ew[VC];
#pragma unroll
        for (int c = 0; c < VC; ++c) ew[c] = scores[min(base + j + kClasses * c, last)];
#pragma unroll
        for (int c = 0; c < VC; ++c) {
            const int pp = base + j + kClasses * c;
            if (c < whole) {
                const float e = ew[c];
                a[0] = a[0] + mul_f16<false>(e, vr[c].x);
                a[1] = a[1] + mul_f16<true>(e, vr[c].x);
                a[2] = a[2] + mul_f16<false>(e, vr[c].y);
                a[3] = a[3] + mul_f16<true>(e, vr[c].y);
                total = total + e;
            } else if (c == whole) {
                const bool ok = pp < nglobal;
                const float e = ew[c];
                const float ev[4] = {mul_f16<false>(e, vr[c].x), mul_f16<true>(e, vr[c].x),
                                     mul_f16<false>(e, vr[c].y), mul_f16<true>(e, vr[c].y)};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float t = a[i] + ev[i];
                    a[i] = ok ? t : a[i];
                }
                const float tt = total + e;
                total = ok ? tt : total;
            }
        }
    }
    if (j == (nglobal & (kClasses - 1))) {  // the newest position closes its class
        const float e = scores[nglobal];
        const __half2 h01 = *reinterpret_cast<const __half2*>(&new_s[1][4 * dq]);
        const __half2 h23 = *reinterpret_cast<const __half2*>(&new_s[1][4 * dq + 2]);
        const float vv[4] = {__low2float(h01), __high2float(h01), __low2float(h23), __high2float(h23)};
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = a[i] + e * vv[i];
        total = total + e;
    }
    *reinterpret_cast<float4*>(&part_s[j][4 * dq]) = make_float4(a[0], a[1], a[2], a[3]);
    if (dq == 0) total_s[j] = total;
    lds_barrier();
    if (tid < kHeadDim && !bad_pos) {
        float o = 0.0f, t = 0.0f;
#pragma unroll
        for (int k = 0; k < kClasses; ++k) {
            o = o + part_s[k][tid];
            t = t + total_s[k];
        }
        p.out[h * kHeadDim + tid] = o * reciprocal(t);
    }
}

hipError_t launch_qkv_attend(const QkvAttendParams& p, int d_model, int prologue, int heads, hipStream_t stream) {
    const size_t lds = sizeof(float) * (size_t)(p.capacity > 0 ? p.capacity : 1);
    if (lds > 96 * 1024 || heads < 1 || d_model != heads * kHeadDim) return hipErrorInvalidValue;
    const dim3 grid(heads), block(512);
    if (d_model == 512) {
        if (prologue == kNorm) rn_launch((qkv_attend_kernel<512, kNorm, 3, 10>), grid, block, lds, stream, p);
        else if (prologue == kEmbedNorm) rn_launch((qkv_attend_kernel<512, kEmbedNorm, 3, 10>), grid, block, lds, stream, p);
        else if (prologue == kEmbedArgmax) rn_launch((qkv_attend_kernel<512, kEmbedArgmax, 3, 10>), grid, block, lds, stream, p);
        else return hipErrorInvalidValue;
    } else if (d_model == 384) {
        if (prologue == kNorm) rn_launch((qkv_attend_kernel<384, kNorm, 3, 10>), grid, block, lds, stream, p);
        else if (prologue == kEmbedNorm) rn_launch((qkv_attend_kernel<384, kEmbedNorm, 3, 10>), grid, block, lds, stream, p);
        else return hipErrorInvalidValue;
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rn
