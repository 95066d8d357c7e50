// rn_whistle.hip — the speech path's own kernels for gfx950: the fp32 stem
// convolutions, per-head norm/rotary/int8 codes, attention with int8 queries,
// keys and values, and the decoder's fused cross-attention.
//
// Replaces crates/whistle/src/frontend.rs:42-133 (FFT, power spectrum, mel
// projection, log, spread and normalisation), stem.rs:39-115 (the two
// conv1d layers of the stem; the second runs as an int8 product over im2col
// rows), encoder.rs:217-297 (the
// attention's integer scores and int8 values) and cross.rs:58-182 (memory,
// apply). Products go
// through the shared int8 kernels (rn_gemm.hip, rn_gemv.hip); the cross
// residual (cross.rs:176-181) is the prologue of the gated FFN's product.
//
// Float orders (identical to the CPU restatement): the first convolution adds
// its taps (k, m) in order into a zero output per (frame, channel); the head
// norm uses the
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

hipError_t launch_stem(const float* mel, const float* conv1, int F, int M, int d, float* h1, hipStream_t stream) {
    if (M < 1 || M > kMaxMels || F < 1 || d < 1) return hipErrorInvalidValue;
    const size_t lds = sizeof(float) * ((size_t)kStemChan * (3 * M + 1) + (size_t)(kStemTime + 2) * M);
    rn_launch(stem_conv_kernel, dim3((F + kStemTime - 1) / kStemTime, (d + kStemChan - 1) / kStemChan), dim3(256), lds,
              stream, mel, conv1, F, M, d, h1);
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
        const float inverse = reciprocal(sqrtf(total / 64.0f + p.eps));
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

// Attention with int8 queries, keys and values (encoder.rs:262-285 for the
// encoder's frames, cross.rs:136-170 for the decoder's cross-attention), for
// one head over at most kMaxFrames frames:
//   score_j = ((float)(q . k_j) * key_scale_j) * query_scale   (exact int32 dot)
//   e_j = fast_exp(score_j - peak)
//   class totals: class c sums e_j over j = c, c+32, ... in order; total adds
//   the classes 0..31; inverse = 1 / total
//   w_j = value_scale_j * (e_j * inverse)
//   out_d = sum over classes 0..31 of (class c's sum over its j, in order, of
//   w_j * (float)v_jd)
// The head's value rows are staged in LDS once per block; scores and weights
// live in LDS. Two block shapes: one query per 1024-thread block (the decoder's
// cross-attention: every load of the block is issued before the first score),
// and tiles of kTileQueries queries per 512-thread block (the encoder: a key
// row or value row loaded once serves the whole tile).
constexpr int kMaxFrames = 1536;
constexpr int kTileQueries = 8;

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void global_void;

// The head's value rows into LDS with global_load_lds_dwordx4 (no registers:
// each lane's 16 bytes land at the wave's LDS base + 16 * lane). Piece i of the
// head is 16-byte quarter i % 4 of frame i / 4 and goes to v_s + 16 i, so a
// wave's 64 pieces are 1 KB of consecutive LDS; frames past the end repeat the
// last frame. The copies count on vmcnt: wait for them before a barrier.
template <int NT>
__device__ __forceinline__ void stage_values(const Int8AttendParams& p, int h, int8_t* v_s) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int c = 0; c < kMaxFrames * 4 / NT; ++c) {
        const int base = NT * c + 64 * wave, id = base + lane, fr = min(id >> 2, p.frames - 1);
        __builtin_amdgcn_global_load_lds((global_void*)(p.vc + ((size_t)fr * p.heads + h) * 64 + (id & 3) * 16),
                                         (lds_void*)(v_s + (size_t)base * 16), 16, 0, 0);
    }
}

// int8 pair (bytes 0, 1 of a 16-bit word) as floats
__device__ __forceinline__ void int8x2_to_float(uint32_t w, float& a, float& b) {
    a = (float)(int)(int8_t)(w & 0xff);
    b = (float)(int)(int8_t)((w >> 8) & 0xff);
}

__global__ __launch_bounds__(1024) void int8_attend_one_kernel(Int8AttendParams p) {
    constexpr int NT = 1024, KP = kMaxFrames / (NT / 4), EP = kMaxFrames / NT + 1;
    __shared__ __align__(16) int8_t v_s[kMaxFrames * 64];
    __shared__ float e_s[kMaxFrames];
    __shared__ float part_s[32][64 + 1];
    __shared__ float tot_s[32];
    __shared__ float red_s[NT / 64];
    const int h = blockIdx.x, q = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int F = p.frames, H = p.heads;
    const int li = tid & 3;
    // 1. every load of the block: the query quarter, the key rows (4 lanes per
    // frame), the value rows as 16-byte pieces, the scales; frames past the end
    // repeat the last frame
    const int4 qq = reinterpret_cast<const int4*>(p.qc + ((size_t)q * H + h) * 64)[li];
    const float qs = p.qs[(size_t)q * H + h];
    int4 kr[KP];
    float ksr[KP];
#pragma unroll
    for (int c = 0; c < KP; ++c) {
        const int fr = min((tid >> 2) + (NT / 4) * c, F - 1);
        kr[c] = reinterpret_cast<const int4*>(p.kc + ((size_t)fr * H + h) * 64)[li];
        ksr[c] = p.ks[(size_t)fr * H + h];
    }
    // six 16-byte value pieces per thread, in named registers (an array this
    // size beside the key rows would be kept in scratch memory)
    static_assert(kMaxFrames * 4 / NT == 6, "six value pieces per thread");
    auto vpiece = [&](int c) -> int4 {
        const int id = tid + NT * c, fr = min(id >> 2, F - 1);
        return reinterpret_cast<const int4*>(p.vc + ((size_t)fr * H + h) * 64)[id & 3];
    };
    const int4 vr0 = vpiece(0), vr1 = vpiece(1), vr2 = vpiece(2), vr3 = vpiece(3), vr4 = vpiece(4), vr5 = vpiece(5);
    float vsr[EP];
#pragma unroll
    for (int c = 0; c < EP; ++c) vsr[c] = p.vs[(size_t)min(tid + NT * c, F - 1) * H + h];
    __builtin_amdgcn_sched_barrier(0);  // every request before the first score

    // 2. scores and the local peak
    float sc[KP];
    float m = -INFINITY;
#pragma unroll
    for (int c = 0; c < KP; ++c) {
        const int fr = (tid >> 2) + (NT / 4) * c;
        int dot = dot16(kr[c], qq, 0);
        dot = dot + dpp_move<0xb1>(dot);
        dot = dot + dpp_move<0x4e>(dot);
        sc[c] = ((float)dot * ksr[c]) * qs;
        if (fr < F) m = fmaxf(m, sc[c]);
    }
    m = wave_max(m);
    // the value rows into LDS (piece id = quarter id % 4 of frame id / 4)
    int4* vp = reinterpret_cast<int4*>(v_s) + tid;
    vp[0] = vr0;
    vp[NT] = vr1;
    vp[2 * NT] = vr2;
    vp[3 * NT] = vr3;
    vp[4 * NT] = vr4;
    vp[5 * NT] = vr5;
    if (lane == 0) red_s[wave] = m;
    __syncthreads();
    float peak = red_s[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) peak = fmaxf(peak, red_s[w]);
    // 3. fast_exp weights, the class totals, then the scaled weights
#pragma unroll
    for (int c = 0; c < KP; ++c) {
        const int fr = (tid >> 2) + (NT / 4) * c;
        if (li == 0 && fr < F) e_s[fr] = fast_exp(sc[c] - peak);
    }
    __syncthreads();
    if (tid < 32) {
        float t = 0.0f;
#pragma unroll
        for (int k = 0; k < kMaxFrames / 32; ++k) {
            const int j = tid + 32 * k;
            if (j < F) t = t + e_s[j];
        }
        tot_s[tid] = t;
    }
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int c = 0; c < 32; ++c) total = total + tot_s[c];
    const float inverse = reciprocal(total);
#pragma unroll
    for (int c = 0; c < EP; ++c) {
        const int j = tid + NT * c;
        if (j < F) e_s[j] = vsr[c] * (e_s[j] * inverse);
    }
    __syncthreads();
    // 4. value sums: thread (class c, dims 2 d2, 2 d2 + 1) walks c, c+32, ...
    const int c = tid >> 5, d2 = tid & 31;
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll 8
    for (int k = 0; k < kMaxFrames / 32; ++k) {
        const int j = c + 32 * k;
        if (j < F) {
            const float w = e_s[j];
            float v0, v1;
            int8x2_to_float(*reinterpret_cast<const uint16_t*>(v_s + j * 64 + 2 * d2), v0, v1);
            a0 = a0 + w * v0;
            a1 = a1 + w * v1;
        }
    }
    part_s[c][2 * d2] = a0;
    part_s[c][2 * d2 + 1] = a1;
    __syncthreads();
    if (tid < 64) {
        float o = 0.0f;
#pragma unroll
        for (int k = 0; k < 32; ++k) o = o + part_s[k][tid];
        p.out[(size_t)q * p.out_stride + h * 64 + tid] = o;
    }
}

// One 512-thread block per (slice, head) runs the tiles slice, slice + slices,
// ... of its head: the head's key rows (registers) and value rows (LDS) are
// loaded once per block and serve every tile it runs; per tile only the
// queries' codes are loaded.
__global__ __launch_bounds__(512) void int8_attend_tile_kernel(Int8AttendParams p, int queries) {
    constexpr int NT = 512, Q = kTileQueries;
    constexpr int KT = kMaxFrames / 16 / (NT / 64);  // 16-frame key tiles per wave
    constexpr int QH = Q / 2;  // queries per pass of the final class sum
    static_assert(Q == 8, "two groups of 4 output rows of the 16-row MFMA operand");
    // LDS: the value rows (96 KB), a tile's scores / weights [frame][query]
    // (48 KB; after the value sums it takes half a tile's class partials)
    __shared__ __align__(16) int8_t v_s[kMaxFrames * 64];
    __shared__ __align__(16) float e_s[kMaxFrames][Q];
    __shared__ float vs_s[kMaxFrames];
    __shared__ float tot_s[Q][32];
    __shared__ float red_s[Q][NT / 64];
    __shared__ float inv_s[Q];
    static_assert(QH * 32 * 64 <= kMaxFrames * Q, "half a tile's partials fit the weight area");
    float(*part_s)[32][64] = reinterpret_cast<float(*)[32][64]>(&e_s[0][0]);
    const int h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int F = p.frames, H = p.heads;
    const int tiles = (queries + Q - 1) / Q;
    // 1. once per block: key rows and scales, value rows (into LDS), value
    // scales; frames past the last repeat the last frame. The keys are held as
    // i8 MFMA fragments: wave w owns frame tiles w, w + 8, ... (16 frames each);
    // lane l holds frame 16 t + l % 16, bytes 8 (l / 16) and 32 + 8 (l / 16)
    const int r16 = lane & 15, kq = lane >> 4;
    long kf[KT][2];
    float kfs[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
        const int fr = min(16 * (wave + (NT / 64) * t) + r16, F - 1);
        const int8_t* row = p.kc + ((size_t)fr * H + h) * 64;
        kf[t][0] = *reinterpret_cast<const long*>(row + 8 * kq);
        kf[t][1] = *reinterpret_cast<const long*>(row + 32 + 8 * kq);
        kfs[t] = p.ks[(size_t)fr * H + h];
    }
    stage_values<NT>(p, h, v_s);
    constexpr int SP = kMaxFrames / NT;
#pragma unroll
    for (int c = 0; c < SP; ++c) vs_s[tid + NT * c] = p.vs[(size_t)min(tid + NT * c, F - 1) * H + h];
    __builtin_amdgcn_s_waitcnt(0);  // this wave's value rows are in LDS
    __syncthreads();

    for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const int q0 = tile * Q;
    // the tile's query fragments: lane l holds query min(l % 16, Q - 1) (rows 8-15
    // of the 16-row operand repeat query 7 and are never read), bytes 8 (l / 16)
    // and 32 + 8 (l / 16); queries past the end repeat the last. Output row
    // 4 (l / 16) + i of lane l is query 4 (l / 16) + i: lanes 0-31 hold the tile.
    long qa0, qa1;
    float qsv[4];
    {
        const int qi = min(q0 + min(r16, Q - 1), queries - 1);
        const int8_t* qrow = p.qc + ((size_t)qi * H + h) * 64;
        qa0 = *reinterpret_cast<const long*>(qrow + 8 * kq);
        qa1 = *reinterpret_cast<const long*>(qrow + 32 + 8 * kq);
#pragma unroll
        for (int i = 0; i < 4; ++i) qsv[i] = p.qs[(size_t)min(q0 + min(4 * kq + i, Q - 1), queries - 1) * H + h];
    }
    // 2. scores for the tile's queries (exact int32 dots on the matrix cores, two
    // 32-byte halves of the head), and their local peaks
    float m[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int t = 0; t < KT; ++t) {
        v4i acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(qa0, kf[t][0], v4i{0, 0, 0, 0}, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(qa1, kf[t][1], acc, 0, 0, 0);
        const int fr = 16 * (wave + (NT / 64) * t) + r16;
        float s[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] = ((float)acc[i] * kfs[t]) * qsv[i];
        if (kq < 2) {
            *reinterpret_cast<float4*>(&e_s[fr][4 * kq]) = make_float4(s[0], s[1], s[2], s[3]);
            if (fr < F)
#pragma unroll
                for (int i = 0; i < 4; ++i) m[i] = fmaxf(m[i], s[i]);
        }
    }
    // the peak of each query over the 16 lanes of its row group (lanes 0-15:
    // queries 0-3, lanes 16-31: queries 4-7)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float mm = m[i];
        mm = fmaxf(mm, __int_as_float(dpp_move<0xb1>(__float_as_int(mm))));
        mm = fmaxf(mm, __int_as_float(dpp_move<0x4e>(__float_as_int(mm))));
        mm = fmaxf(mm, __int_as_float(dpp_move<0x141>(__float_as_int(mm))));
        mm = fmaxf(mm, __int_as_float(dpp_move<0x140>(__float_as_int(mm))));
        if (lane == 0 || lane == 16) red_s[4 * kq + i][wave] = mm;
    }
    __syncthreads();
    // 3. fast_exp weights (element (frame, query) = (e / Q, e % Q)); frames past
    // the last get weight 0, so the loops below run over every frame slot: an
    // exact +0 addend leaves a running sum that started at +0 unchanged (and
    // those slots' value rows repeat the last frame, so they are finite)
    static_assert((kMaxFrames * Q) % NT == 0, "whole weight passes");
    {
        const int i = tid % Q;  // NT is a multiple of Q: each thread keeps one query
        float peak = red_s[i][0];
#pragma unroll
        for (int w = 1; w < NT / 64; ++w) peak = fmaxf(peak, red_s[i][w]);
#pragma unroll 4
        for (int e = tid; e < kMaxFrames * Q; e += NT) {
            float& x = e_s[e / Q][i];
            x = e / Q < F ? fast_exp(x - peak) : 0.0f;
        }
    }
    __syncthreads();
    if (tid < Q * 32) {  // class totals: thread (query i, class c)
        const int i = tid >> 5, c = tid & 31;
        float t = 0.0f;
#pragma unroll
        for (int k = 0; k < kMaxFrames / 32; ++k) t = t + e_s[c + 32 * k][i];
        tot_s[i][c] = t;
    }
    __syncthreads();
    if (tid < Q) {
        float total = 0.0f;
#pragma unroll
        for (int c = 0; c < 32; ++c) total = total + tot_s[tid][c];
        inv_s[tid] = reciprocal(total);
    }
    __syncthreads();
    {
        const int i = tid % Q;
        const float inverse = inv_s[i];
#pragma unroll 4
        for (int e = tid; e < kMaxFrames * Q; e += NT) {
            const int j = e / Q;
            e_s[j][i] = vs_s[j] * (e_s[j][i] * inverse);
        }
    }
    __syncthreads();
    // 4. value sums: thread (class c, dims 4 dq..4 dq + 3) for every query of the tile
    const int c = tid >> 4, dq = tid & 15;
    float a[Q][4];
#pragma unroll
    for (int i = 0; i < Q; ++i)
#pragma unroll
        for (int d = 0; d < 4; ++d) a[i][d] = 0.0f;
#pragma unroll 4
    for (int k = 0; k < kMaxFrames / 32; ++k) {
        const int j = c + 32 * k;
        const uint32_t raw = *reinterpret_cast<const uint32_t*>(v_s + j * 64 + 4 * dq);
        float v[4];
        int8x2_to_float(raw, v[0], v[1]);
        int8x2_to_float(raw >> 16, v[2], v[3]);
        const float4 w0 = *reinterpret_cast<const float4*>(&e_s[j][0]);
        const float4 w1 = *reinterpret_cast<const float4*>(&e_s[j][4]);
        const float w[Q] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int i = 0; i < Q; ++i)
#pragma unroll
            for (int d = 0; d < 4; ++d) a[i][d] = a[i][d] + w[i] * v[d];
    }
    // 5. out = the class partials added in class order, half a tile at a time
    // through the weight area (the value rows stay for the next tile)
    static_assert(NT == QH * 2 * 64, "one output per thread of each half pass");
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        __syncthreads();  // the area's previous contents are read
#pragma unroll
        for (int i = 0; i < QH; ++i) {
            const float* ai = a[QH * half + i];
            *reinterpret_cast<float4*>(&part_s[i][c][4 * dq]) = make_float4(ai[0], ai[1], ai[2], ai[3]);
        }
        __syncthreads();
        if (tid < QH * 64) {
            const int i = tid >> 6, d = tid & 63;
            float o = 0.0f;
#pragma unroll
            for (int k = 0; k < 32; ++k) o = o + part_s[i][k][d];
            const int qi = q0 + QH * half + i;
            if (qi < queries) p.out[(size_t)qi * p.out_stride + h * 64 + d] = o;
        }
    }
    __syncthreads();  // the partials are read before the next tile's scores
    }
}

hipError_t launch_int8_attend(const Int8AttendParams& p, int queries, hipStream_t stream) {
    if (queries <= 0) return hipSuccess;
    if (p.frames < 1 || p.frames > kMaxFrames || p.heads < 1) return hipErrorInvalidValue;
    if (queries < kTileQueries) {
        rn_launch(int8_attend_one_kernel, dim3(p.heads, queries), dim3(1024), 0, stream, p);
    } else {
        // one block per CU: as few slices per head as keep the rounds of tiles per
        // CU at their minimum
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            cus = 256;
        const int tiles = (queries + kTileQueries - 1) / kTileQueries;
        const long work = (long)tiles * p.heads;
        const int rounds = (int)((work + cus - 1) / cus);
        const int slices = (tiles + rounds - 1) / rounds;
        rn_launch(int8_attend_tile_kernel, dim3(slices, p.heads), dim3(512), 0, stream, p, queries);
    }
    return hipGetLastError();
}

// The decoder's cross-attention of one token (cross.rs:126-170 up to the
// attention output) in 1024-thread blocks, kCrossGroups per head: block b
// serves head b % 8 and position-class group g = b / 8 (classes
// kGroupClasses g .. kGroupClasses g + kGroupClasses - 1). Blocks are dealt to
// the XCDs round-robin, so a head's blocks share one L2 for the key rows every
// one of them reads; blocks of heads the model lacks exit at once. One block
// per head would be bound by its value sums (about 4600 wave instructions
// through one CU); split eight ways, the redundant part (keys, scores, softmax
// total) costs less than the split saves. The block's loads (about 150 KB,
// the bound of the front half: one CU takes about 64 bytes a clock) are all
// requested at the start, each by the wave that uses it, and no barrier
// separates the q product from them:
//   1. wave 0 requests x, the cross gains, the q rows' scales and the q_norm
//      gains; waves 1..kProductWaves the head's 64 rows of the cross q matrix;
//      each thread t of the memory waves (kProductWaves + 1 .. 15) the key rows
//      of frames t and t + 768, a 16-byte piece of the group's value rows and
//      a value scale;
//   2. wave 0: the zero-centred norm of x (eight-lane sum of ops.rs:7-17) and
//      its int8 codes (ops.rs:103-118) into LDS, then it raises an LDS flag;
//   3. the product waves, once the flag is up: v_dot4 group sums (lane pairs
//      joined into 32-code groups), each then counting itself done in LDS;
//      wave 1, once all have: lane r runs row r's panel epilogue
//      fmaf(acc, sW * sx, total) (panel.rs:184-188), then the head's
//      zero-centred q norm with the q_norm gains, its int8 codes and scale
//      times 1/sqrt(64) (encoder.rs:239-244);
//   4. the memory waves: scores ((float)(q . k) * key_scale) * query_scale
//      (exact int32 dot), the peak, fast_exp(score - peak) for every frame (0
//      past the last);
//   5. wave 0: the 32 class totals (frames c, c+32, ... in order), their sum
//      over classes 0..31, inverse = 1/total, and the group's weights
//      value_scale * (e * inverse) (ops.rs:92-101, encoder.rs:278-285), while
//      waves 1..kGroupClasses convert their class's int8 values to floats;
//   6. those waves, lane = dim: the weighted value sum over the class's frames
//      in order, stored as part[class][64 h + lane].
// Frames past the last add exact zeros: a weight of +0 adds +-0 to a running
// sum that starts at +0, which leaves it unchanged, so the loops need no
// bounds. Value row r of group g holds frame
// 32 (r / kGroupClasses) + kGroupClasses g + r % kGroupClasses.
constexpr int kCrossGroups = 8;
constexpr int kGroupClasses = 32 / kCrossGroups;
constexpr int kCrossRows = kMaxFrames / kCrossGroups;  // value rows per block
constexpr int kProductWaves = 3;                        // waves 1..3 take the q product

template <int K>
__global__ __launch_bounds__(1024) void cross_attend_kernel(CrossAttendParams p) {
    constexpr int NT = 1024;
    constexpr int G = K / kGroup, CPR = K / 16, CHUNKS = kWave * CPR;
    constexpr int LW = kProductWaves * kWave;   // threads of the q product (waves 1..kProductWaves)
    constexpr int NLW = (CHUNKS + LW - 1) / LW;
    constexpr int MW0 = 1 + kProductWaves;      // first memory wave
    constexpr int MT = NT - MW0 * kWave;        // memory threads
    constexpr int E = K / kWave;
    constexpr int FPC = kMaxFrames / 32;  // frame slots per class
    static_assert(kMaxFrames == 2 * MT, "two key rows per memory thread");
    static_assert(kCrossRows * 4 <= MT && kCrossRows <= MT && kCrossRows % kWave == 0,
                  "one value piece and one value scale per memory thread, whole weight rows");
    static_assert(kGroupClasses + 1 <= NT / kWave, "value-sum waves besides wave 0");
    static_assert(E % 2 == 0 && G % 4 == 0 && CPR % 2 == 0, "float pairs, scale quads, code pairs");
    __shared__ __align__(16) int8_t v_s[kCrossRows * 64];
    __shared__ float e_s[kMaxFrames];
    __shared__ float w_s[kCrossRows];
    __shared__ __align__(16) int8_t xq_s[K];
    __shared__ __align__(16) float sq_s[K];
    __shared__ __align__(16) int acc_s[kWave * G];
    __shared__ __align__(16) int8_t qc_s[kWave];
    __shared__ float red_s[NT / kWave];
    __shared__ __align__(16) float4 sw_s[kWave][G / 4];
    __shared__ float qg_s[kWave];
    __shared__ float sx_s, qs_s;
    __shared__ int codes_ready_s, rows_done_s;  // LDS flags between waves 0 and 1..kProductWaves

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x & 7, g = blockIdx.x >> 3;
    const int H = p.heads, F = p.frames;
    if (h >= H) return;  // uniform over the block, before any barrier
    auto frame_of_row = [&](int r) -> int {
        return 32 * (r / kGroupClasses) + kGroupClasses * g + r % kGroupClasses;
    };
    if (tid == 0) {
        codes_ready_s = 0;
        rows_done_s = 0;
    }
    __syncthreads();  // the flags start at zero before any wave waits on them

    // 1. requests: wave 0 the prologue inputs (and the q rows' scales and the
    // q_norm gains, staged in LDS for wave 1); the product waves the head's 64
    // rows of the cross q matrix; the memory waves the key rows of frames t and
    // t + MT (t = tid - 64 MW0), a 16-byte piece of the group's value rows and a
    // value scale. Frames past the last repeat the last frame; offsets fit 32
    // bits (at most 1536 x 8 x 64 bytes).
    // The product waves' chunks and the memory waves' rows share one register
    // array r: every variable set in one branch of this phase stays live past
    // it, so separate arrays would each take registers in every wave.
    typedef float v4f __attribute__((ext_vector_type(4)));  // kept in registers, unlike float4 arrays
    constexpr int RW = NLW > 9 ? NLW : 9;  // product: r[0..NLW); memory: keys r[0..8), values r[8]
    v4i r[RW];
    v4f sv[G / 4];
    float qgain = 0.0f;
    float v[E], gv[E];
    const int t = tid - MW0 * kWave;  // memory thread index (memory waves only)
    float ks0 = 0.0f, ks1 = 0.0f, vsr = 0.0f;
    if (wave == 0) {
        load_floats<E>(p.x + lane * E, v);
        load_floats<E>(p.gain + lane * E, gv);
        const v4f* src = reinterpret_cast<const v4f*>(p.sW + (size_t)(kWave * h + lane) * G);
#pragma unroll
        for (int i = 0; i < G / 4; ++i) sv[i] = src[i];
        qgain = p.q_gain[lane];
    } else if (wave < MW0) {
        // chunk c = LW jj + (tid - 64): chunk c % CPR of head row c / CPR
#pragma unroll
        for (int jj = 0; jj < NLW; ++jj) {
            const int c = min(LW * jj + tid - kWave, CHUNKS - 1);
            r[jj] = *reinterpret_cast<const v4i*>(p.W + (size_t)(kWave * h + c / CPR) * K + (c % CPR) * 16);
        }
    } else {
        const uint32_t fh0 = (uint32_t)(min(t, F - 1) * H + h);
        const uint32_t fh1 = (uint32_t)(min(MT + t, F - 1) * H + h);
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = reinterpret_cast<const v4i*>(p.kc + fh0 * 64u)[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) r[4 + i] = reinterpret_cast<const v4i*>(p.kc + fh1 * 64u)[i];
        ks0 = p.ks[fh0];
        ks1 = p.ks[fh1];
        r[8] = *reinterpret_cast<const v4i*>(p.vc + (uint32_t)(min(frame_of_row(t >> 2), F - 1) * H + h) * 64u +
                                             (uint32_t)(t & 3) * 16u);
        vsr = p.vs[(uint32_t)(min(frame_of_row(min(t, kCrossRows - 1)), F - 1) * H + h)];
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. wave 0: the input's norm and int8 codes; then it raises codes_ready_s
    if (wave == 0) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int idx = lane * E + e;
            sq_s[(idx % 8) * (K / 8) + idx / 8] = v[e] * v[e];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float s = 0.0f;
        if (lane < 8) {
            // the run in quarters of four float4s (all memory loads are still
            // in flight, so registers are short here)
            const float4* run = reinterpret_cast<const float4*>(sq_s + lane * (K / 8));
#pragma unroll
            for (int c0 = 0; c0 < K / 32; c0 += 4) {
                float4 t[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) t[c] = run[c0 + c];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    s = s + t[c].x;
                    s = s + t[c].y;
                    s = s + t[c].z;
                    s = s + t[c].w;
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        float total = sum_lanes_0_to_7(s);
        total = total + 0.0f;  // the (empty) tail of ops.rs:15-16
        const float inverse = reciprocal(sqrtf(total / (float)K + p.eps));
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = ((1.0f + gv[e]) * v[e]) * inverse;
        float peak = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) peak = fmaxf(peak, fabsf(v[e]));
        peak = wave_max_nonneg(peak);
        const float sx = int8_scale_from_peak(peak);
        float y[E];
        quotients<E>(v, sx, y);
#pragma unroll
        for (int e = 0; e < E; ++e) xq_s[lane * E + e] = (int8_t)code_of_quotient(y[e]);
        if (lane == 0) sx_s = sx;
#pragma unroll
        for (int i = 0; i < G / 4; ++i) sw_s[lane][i] = make_float4(sv[i].x, sv[i].y, sv[i].z, sv[i].w);
        qg_s[lane] = qgain;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0) __hip_atomic_store(&codes_ready_s, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }

    // 3. the head's q rows: the product waves wait for the codes on the LDS flag
    // (not a barrier: the memory waves may still be issuing their requests), add
    // their group sums, and count themselves done; wave 1 then runs the row
    // epilogues and the head's q codes. Both waits end once the waves they wait
    // for have passed the flag writes above and below, which no branch skips;
    // the spin is bounded all the same.
    if (wave >= 1 && wave < MW0) {
        for (int spin = 0; spin < (1 << 22); ++spin) {
            if (__hip_atomic_load(&codes_ready_s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0) break;
            __builtin_amdgcn_s_sleep(1);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
#pragma unroll
        for (int jj = 0; jj < NLW; ++jj) {
            const int c = LW * jj + tid - kWave;
            const int4 xc = *reinterpret_cast<const int4*>(xq_s + (min(c, CHUNKS - 1) % CPR) * 16);
            int part = dot16(r[jj], xc, 0);
            part = part + dpp_move<0xb1>(part);  // the pair partner (lane ^ 1: chunk c ^ 1)
            if ((tid & 1) == 0 && c < CHUNKS) acc_s[(c / CPR) * G + (c % CPR) / 2] = part;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0) __hip_atomic_fetch_add(&rows_done_s, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (wave == 1) {
        for (int spin = 0; spin < (1 << 22); ++spin) {
            if (__hip_atomic_load(&rows_done_s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == kProductWaves)
                break;
            __builtin_amdgcn_s_sleep(1);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        const float sx = sx_s;
        const int4* arow = reinterpret_cast<const int4*>(acc_s + lane * G);
        float q = 0.0f;
#pragma unroll
        for (int i = 0; i < G / 4; ++i) {
            const int4 a4 = arow[i];
            const float4 s4 = sw_s[lane][i];
            q = fmaf((float)a4.x, s4.x * sx, q);
            q = fmaf((float)a4.y, s4.y * sx, q);
            q = fmaf((float)a4.z, s4.z * sx, q);
            q = fmaf((float)a4.w, s4.w * sx, q);
        }
        const float qgain = qg_s[lane];
        // per-head q norm (lane j < 8 of the eight-lane sum gathers j, j+8, ...)
        const float sq = q * q;
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) s = s + __shfl(sq, 8 * c + (lane & 7), kWave);
        float total = sum_lanes_0_to_7(s);
        total = total + 0.0f;
        const float inverse = reciprocal(sqrtf(total / 64.0f + p.eps));
        q = ((1.0f + qgain) * q) * inverse;
        const float scale = int8_scale_from_peak(wave_max(fabsf(q)));
        float y;
        quotients<1>(&q, scale, &y);
        qc_s[lane] = (int8_t)code_of_quotient(y);
        if (lane == 0) qs_s = scale * (1.0f / sqrtf(64.0f));
    }
    __syncthreads();

    // 4. the memory waves: scores of frames t and t + MT and their peak; the
    // group's value rows and scales into LDS
    float sc0 = 0.0f, sc1 = 0.0f, m = -INFINITY;
    if (wave >= MW0) {
        const float qs = qs_s;
        int d0 = 0, d1 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int4 qv = reinterpret_cast<const int4*>(qc_s)[i];
            d0 = dot16(r[i], qv, d0);
            d1 = dot16(r[4 + i], qv, d1);
        }
        sc0 = ((float)d0 * ks0) * qs;
        sc1 = ((float)d1 * ks1) * qs;
        if (t < F) m = sc0;
        if (MT + t < F) m = fmaxf(m, sc1);
        reinterpret_cast<v4i*>(v_s)[t] = r[8];
        if (t < kCrossRows) w_s[t] = frame_of_row(t) < F ? vsr : 0.0f;  // value scales for now
    }
    m = wave_max(m);
    if (lane == 0) red_s[wave] = m;
    __syncthreads();
    float peak = red_s[0];
#pragma unroll
    for (int i = 1; i < NT / kWave; ++i) peak = fmaxf(peak, red_s[i]);
    if (wave >= MW0) {
        e_s[t] = t < F ? fast_exp(sc0 - peak) : 0.0f;
        e_s[MT + t] = MT + t < F ? fast_exp(sc1 - peak) : 0.0f;
    }
    __syncthreads();

    // 5. wave 0: class totals, total, and the group's weights; the value-sum
    // waves meanwhile take their int8 values out of LDS as floats
    float vf[FPC];
    const int cls = wave - 1;  // the value-sum waves' class within the group
    if (wave == 0) {
        float t[FPC];
#pragma unroll
        for (int k = 0; k < FPC; ++k) t[k] = e_s[(lane & 31) + 32 * k];
        float ct = 0.0f;
#pragma unroll
        for (int k = 0; k < FPC; ++k) ct = ct + t[k];
        float total = 0.0f;
#pragma unroll
        for (int c = 0; c < 32; ++c) total = total + lane_float(ct, c);
        const float inverse = reciprocal(total);
#pragma unroll
        for (int k = 0; k < kCrossRows / kWave; ++k) {
            const int r = lane + kWave * k;
            w_s[r] = w_s[r] * (e_s[frame_of_row(r)] * inverse);
        }
    } else if (cls < kGroupClasses) {
#pragma unroll
        for (int k = 0; k < FPC; ++k) vf[k] = (float)v_s[(kGroupClasses * k + cls) * 64 + lane];
    }
    __syncthreads();

    // 6. the value sums of class kGroupClasses g + cls (lane = dim), frames in order
    if (wave >= 1 && cls < kGroupClasses) {
        float a = 0.0f;
#pragma unroll
        for (int k = 0; k < FPC; ++k) a = a + w_s[kGroupClasses * k + cls] * vf[k];
        p.part[(size_t)(kGroupClasses * g + cls) * (H * 64) + h * 64 + lane] = a;
    }
}

hipError_t launch_cross_attend(const CrossAttendParams& p, int d_model, hipStream_t stream) {
    if (p.frames < 1 || p.frames > kMaxFrames || p.heads < 1 || p.heads > 8 || d_model != p.heads * 64)
        return hipErrorInvalidValue;
    const dim3 grid(8 * kCrossGroups);
    switch (d_model) {
        case 384:
            rn_launch(cross_attend_kernel<384>, grid, dim3(1024), 0, stream, p);
            break;
        case 512:
            rn_launch(cross_attend_kernel<512>, grid, dim3(1024), 0, stream, p);
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

namespace rn {

// Frontend::log_mel (frontend.rs:72-102) up to the log: one 256-thread block per
// frame. The windowed samples go straight to their bit-reversed slots (the swap
// loop of frontend.rs:44-50 leaves slot i holding input rev(i)); the
// butterflies of each span run one per thread with the reference's float
// operations (frontend.rs:52-66); the power spectrum, then per mel the
// projection summed bin by bin and ln(value + FLOOR).
__global__ __launch_bounds__(256) void log_mel_kernel(FrontendParams p, const float* samples, int n, float* data) {
    extern __shared__ __align__(16) float fft_s[];
    float* re = fft_s;
    float* im = fft_s + p.fft_size;
    float* power = fft_s + 2 * p.fft_size;
    const int tid = threadIdx.x, frame = blockIdx.x, size = p.fft_size;
    const int bins = size / 2 + 1, half = p.window / 2;
    for (int i = tid; i < size; i += 256) {
        re[i] = 0.0f;
        im[i] = 0.0f;
    }
    __syncthreads();
    for (int pos = tid; pos < p.window && pos < size; pos += 256) {
        const long long source = (long long)frame * p.hop + pos - half;
        if (source >= 0 && source < n) re[__brev((unsigned)pos) >> (32 - p.log2_size)] = samples[source] * p.window_gain[pos];
    }
    for (int span = 1; span < size; span *= 2) {
        __syncthreads();
        const int stride = size / (span * 2);
        for (int j = tid; j < size / 2; j += 256) {
            const int offset = j % span, a = (j / span) * 2 * span + offset, b = a + span;
            const float c = p.twiddle_cos[offset * stride], s = p.twiddle_sin[offset * stride];
            const float tr = re[b] * c - im[b] * s;
            const float ti = re[b] * s + im[b] * c;
            re[b] = re[a] - tr;
            im[b] = im[a] - ti;
            re[a] = re[a] + tr;
            im[a] = im[a] + ti;
        }
    }
    __syncthreads();
    for (int bin = tid; bin < bins; bin += 256) power[bin] = re[bin] * re[bin] + im[bin] * im[bin];
    __syncthreads();
    for (int m = tid; m < p.mels; m += 256) {
        float row = 0.0f;
        for (int bin = 0; bin < bins; ++bin) row = row + power[bin] * p.mel_weights[(size_t)bin * p.mels + m];
        data[(size_t)frame * p.mels + m] = libm_logf(row + 5.9604645e-8f);  // FLOOR, frontend.rs:3
    }
}

// Frontend::spread and normalise (frontend.rs:104-133), one wave per mel: the
// wave stages the mel's column in LDS (4096 frames at a time, every load
// independent), lane 0 adds the mean and the squared deviations over the valid
// frames in order (from -0.0, as Iterator::sum does), and the wave writes the
// normalised column (0 past the valid frames). dev[m] keeps the spread's
// per-mel deviation for spread_kernel.
constexpr int kColumnChunk = 4096;

__global__ __launch_bounds__(64) void normalise_mels_kernel(float* data, int frames, int valid, int mels, float* dev) {
    __shared__ __align__(16) float col_s[kColumnChunk];
    __shared__ float stats_s[2];
    const int lane = threadIdx.x, m = blockIdx.x;
    auto column_sum = [&](float mean, bool squares) -> float {
        float total = -0.0f;
        for (int f0 = 0; f0 < valid; f0 += kColumnChunk) {
            const int rows = min(kColumnChunk, valid - f0);
            for (int r0 = 0; r0 < rows; r0 += 64 * 16) {  // sixteen loads in flight a lane
                float t[16];
#pragma unroll
                for (int k = 0; k < 16; ++k) t[k] = data[(size_t)(f0 + min(r0 + 64 * k + lane, rows - 1)) * mels + m];
#pragma unroll
                for (int k = 0; k < 16; ++k)
                    if (r0 + 64 * k + lane < rows) col_s[r0 + 64 * k + lane] = t[k];
            }
            __syncthreads();
            if (squares) {  // the squared deviations in parallel; only their sum is sequential
                for (int r = lane; r < rows; r += 64) {
                    const float d = col_s[r] - mean;
                    col_s[r] = d * d;
                }
                __syncthreads();
            }
            if (lane == 0) {
                int r = 0;
                for (; r + 16 <= rows; r += 16) {  // sixteen values read ahead, added in order
                    float4 q[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) q[i] = reinterpret_cast<const float4*>(col_s + r)[i];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        total = total + q[i].x;
                        total = total + q[i].y;
                        total = total + q[i].z;
                        total = total + q[i].w;
                    }
                }
                for (; r < rows; ++r) total = total + col_s[r];
            }
            __syncthreads();
        }
        return total;
    };
    const float sum = column_sum(0.0f, false);
    if (lane == 0) stats_s[0] = sum / (float)(valid > 1 ? valid : 1);  // = sum / valid whenever valid >= 1
    __syncthreads();
    const float mean = stats_s[0];
    const float sq = column_sum(mean, true);
    if (lane == 0) {
        dev[m] = valid >= 2 ? sqrtf(sq / (float)(valid - 1)) : 0.0f;
        const float denominator = fmaxf((float)(valid > 1 ? valid : 1) - 1.0f, 1.0f);
        stats_s[1] = 1.0f / (sqrtf(sq / denominator) + 1e-5f);  // NORMALISER_EPSILON, frontend.rs:4
    }
    __syncthreads();
    const float scale = stats_s[1];
    for (int f = lane; f < frames; f += 64) {
        float* slot = data + (size_t)f * mels + m;
        *slot = f < valid ? (*slot - mean) * scale : 0.0f;
    }
}

// frontend.rs:110-115: the per-mel deviations added in mel order, over mels.
__global__ void spread_kernel(const float* dev, int valid, int mels, float* spread) {
    if (threadIdx.x != 0) return;
    float total = 0.0f;
    for (int i = 0; i < mels; ++i) total = total + dev[i];
    *spread = valid >= 2 ? total / (float)mels : 0.0f;
}

hipError_t launch_log_mel(const FrontendParams& p, const float* samples, int n, float* data, float* spread,
                          hipStream_t stream) {
    if (n < 0 || p.mels < 1 || p.mels > 256 || p.fft_size < 2 || p.fft_size > 4096 || p.hop < 1)
        return hipErrorInvalidValue;
    const int frames = n / p.hop + 1, valid = n / p.hop;
    const size_t lds = sizeof(float) * (2 * (size_t)p.fft_size + p.fft_size / 2 + 1);
    rn_launch(log_mel_kernel, dim3(frames), dim3(256), lds, stream, p, samples, n, data);
    rn_launch(normalise_mels_kernel, dim3(p.mels), dim3(64), 0, stream, data, frames, valid, p.mels, spread + 1);
    rn_launch(spread_kernel, dim3(1), dim3(64), 0, stream, spread + 1, valid, p.mels, spread);
    return hipGetLastError();
}

}  // namespace rn
