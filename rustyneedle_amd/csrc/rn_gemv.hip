// rn_gemv.hip — batch-1 quantised products for gfx950 (the decode GEMVs).
//
// Replaces the CPU row products of crates/kernels (matrix.rs:155-202 fan-out,
// panel.rs:153-197 panel tile, neon.rs:126-183 row_dot) for int8 codes with one
// fp32 scale per 32 columns.
//
// Shape of one block: a single wave (64 lanes) owns ROWS consecutive rows.
//   1. Every lane issues its 128-bit weight loads first (NL loads of 16 codes),
//      and the block stages its ROWS x G scales in LDS; the HBM latency of
//      those loads overlaps the prologue.
//   2. Prologue: the block reads the input vector and quantises it per row
//      (ops.rs:112-118), optionally after the zero-centred RMSNorm
//      (ops.rs:44-50, sum-of-squares tree of ops.rs:7-17) and, for layer 0 of a
//      decode step, after gathering the embedding row of the current token.
//      Every block repeats this small prologue instead of synchronising the
//      grid: the vector is 2-8 KB and stays in L2.
//   3. v_dot4_i32_i8 over the 16 codes of each load; lane pairs hold the two
//      halves of one 32-code group and are added exactly with a lane shuffle.
//   4. Group accumulators go through LDS to lane r, which runs row r's epilogue
//      sequentially over groups (panel form fmaf(acc, sW*sx, total), or plane
//      form total + (acc*sW)*sx), then the fused tail: store, residual add,
//      silu(gate)*up, or logits + on-device argmax.
#include "rn_device.hpp"
#include "rn_internal.hpp"

namespace rn {

template <int K, int ROWS, int PRO, int EPI, int FORM>
__global__ __launch_bounds__(64) void gemv_kernel(GemvParams p) {
    constexpr int G = K / kGroup;                       // groups per row
    constexpr int CPR = K / 16;                         // 16-byte chunks per row
    constexpr int NL = ROWS * CPR / 64;                 // load instructions per lane
    constexpr int E = K / 64;                           // input values per lane in the prologue
    constexpr int H = ROWS / 2;
    static_assert((ROWS * CPR) % 64 == 0, "rows per block must cover whole load instructions");
    static_assert(E % 2 == 0 && G % 4 == 0, "input pairs per lane, scale quads per row");
    static_assert(EPI != kSilu || ROWS % 2 == 0, "silu blocks pair gate and up rows");
    static_assert(ROWS <= 64, "one lane per row in the epilogue");

    constexpr bool NORM = PRO == kNorm || PRO == kEmbedNorm || PRO == kCrossNorm;
    __shared__ __align__(16) int8_t xq_s[K];
    __shared__ __align__(16) int acc_s[ROWS * G];
    __shared__ __align__(16) float sq_s[NORM ? K : 4];

    const int lane = threadIdx.x;

    // Memory-level order matters: loads complete in issue order for the wait
    // counter, so the prologue inputs go first, then the weights, then the
    // row scales; the prologue then waits only for its own inputs.
    // The block's segment is its grid row; a segment with fewer blocks than the
    // grid's width leaves its last blocks with rows past its end, which load
    // the last row again and store nothing. Its fields are read with the input
    // pointers (one argument round trip).
    const Segment sg = p.seg[blockIdx.y];
    const int blk = (int)blockIdx.x;
    __builtin_amdgcn_sched_barrier(0);
    // 1a. prologue inputs
    float v[E];
    float gv[NORM ? E : 1];
    if constexpr (PRO == kEmbedNorm) {
        uint32_t token = p.state->token;
        if (token >= (uint32_t)p.vocab) {
            if (lane == 0 && blockIdx.x == 0) atomicOr(&p.state->error, 1);
            token = 0;
        }
        const int8_t* er = p.embW + (size_t)token * K + lane * E;
#pragma unroll
        for (int e = 0; e < E; ++e)
            v[e] = ((float)er[e] * p.embS[(size_t)token * G + (lane * E + e) / kGroup]) * p.embed_scale;
    } else if constexpr (PRO == kClassSum) {
        // element i is the sum of the 32 class partials x[c][i] in class order
        // (tree T3 of the cross-attention's value sums); all 32 rows requested
        // before the first add
        float t[32][E];
#pragma unroll
        for (int c = 0; c < 32; ++c) load_floats<E>(p.x + (size_t)c * K + lane * E, t[c]);
#pragma unroll
        for (int e = 0; e < E; ++e) {
            v[e] = 0.0f;
#pragma unroll
            for (int c = 0; c < 32; ++c) v[e] = v[e] + t[c][e];
        }
    } else if constexpr (PRO != kCodes) {
        load_floats<E>(p.x + lane * E, v);
    }
    constexpr int CE = PRO == kCrossNorm ? E : 1;
    float av[CE], pg[CE];
    if constexpr (PRO == kCrossNorm) {
        load_floats<E>(p.attended + lane * E, av);
        load_floats<E>(p.post_gain + lane * E, pg);
    }
    if constexpr (NORM) load_floats<E>(p.gain + lane * E, gv);
    // the inputs are requested before the weights
    __builtin_amdgcn_sched_barrier(0);


    auto row_of = [&](int rr) -> int {
        if constexpr (EPI == kSilu) return rr < H ? blk * H + rr : p.half_rows + blk * H + (rr - H);
        else return blk * ROWS + rr;
    };
    auto row_valid = [&](int rr) -> bool {
        if constexpr (EPI == kSilu) return blk * H + (rr < H ? rr : rr - H) < p.half_rows;
        else return blk * ROWS + rr < sg.rows;
    };
    // The row a lane loads from: past the end of the matrix it re-reads the last
    // row (never stored), so loads need no condition.
    auto row_load = [&](int rr) -> int {
        if constexpr (EPI == kSilu) {
            const int i = min(blk * H + (rr < H ? rr : rr - H), p.half_rows - 1);
            return rr < H ? i : p.half_rows + i;
        } else {
            return min(blk * ROWS + rr, sg.rows - 1);
        }
    };
    // load j of a lane covers chunk (64 j + lane) of the block's rows, in row-major order
    auto load_row = [&](int j) -> int { return (64 * j + lane) / CPR; };
    auto load_chunk = [&](int j) -> int { return (64 * j + lane) % CPR; };

    // 1b. weights: unconditional loads (a branch around a load would make the
    // wait counter unknowable and force a full wait)
    int4 w[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j)
        w[j] = *reinterpret_cast<const int4*>(sg.W + (size_t)row_load(load_row(j)) * K + load_chunk(j) * 16);
    // 1c. lane r < ROWS holds the G scales of its row, and for the residual
    // add the row's current value, requested now rather than after the
    // epilogue (each row belongs to one block, which reads it before writing it)
    float4 sv[G / 4];
    const bool mine = lane < ROWS && row_valid(lane);
    {
        const float4* src = reinterpret_cast<const float4*>(sg.sW + (size_t)row_load(min(lane, ROWS - 1)) * G);
#pragma unroll
        for (int i = 0; i < G / 4; ++i) sv[i] = src[i];
    }
    float residual_in = 0.0f;
    if constexpr (EPI == kResidual) {
        const int rr = row_load(min(lane, ROWS - 1));
        residual_in = p.res != nullptr ? p.res[rr] : sg.y[rr];
    }
    // keep the scheduler from sinking those loads below the prologue
    __builtin_amdgcn_sched_barrier(0);

    // 2. prologue: the int8 codes of the input vector and its scale
    float sx;
    int4 xc[NL];
    if constexpr (PRO == kCodes) {
        sx = p.xs[0];
#pragma unroll
        for (int j = 0; j < NL; ++j) xc[j] = *reinterpret_cast<const int4*>(p.xq + load_chunk(j) * 16);
    } else {
        // ops.rs:7-17 for the E values of every lane: lane j of eight sums elements
        // j, j+8, j+16, ... in index order. Squares are stored transposed
        // (strided lane j's run is contiguous) so each of the eight lanes reads
        // its run with 128-bit reads. Returns 1 / sqrt(mean square + eps).
        // GAINED: vals become the gained values m = (1 + g) x and *peak their
        // wave peak |m|, formed while the squares' LDS writes complete (the
        // normed value is fl(m * inverse) with inverse > 0 and rounding is
        // monotone, so the normed peak is fl(peak(|m|) * inverse)).
        auto norm_inverse = [&](float* vals, const float* gains, float* peak) -> float {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const int idx = lane * E + e;
                sq_s[(idx % 8) * (K / 8) + idx / 8] = vals[e] * vals[e];
            }
            if (gains != nullptr) {
                float pk = 0.0f;
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    vals[e] = (1.0f + gains[e]) * vals[e];
                    pk = fmaxf(pk, fabsf(vals[e]));
                }
                *peak = wave_max_nonneg(pk);
            }
            wave_lds_sync();
            float s = 0.0f;
            if (lane < 8) {
                // the whole run requested before the first add (one LDS round
                // trip, not one per read)
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
            const float mean_square = total / (float)K;
            return reciprocal(sqrtf(mean_square + p.eps));
        };
        if constexpr (PRO == kEmbedNorm) {
            if (blockIdx.x == 0)
#pragma unroll
                for (int e = 0; e < E; ++e) p.x_out[lane * E + e] = v[e];
        }
        if constexpr (PRO == kCrossNorm) {
            // cross.rs:176-181: x += cross_gain * zero_centred_norm(attended, post_gain)
            const float inverse = norm_inverse(av, nullptr, nullptr);
#pragma unroll
            for (int e = 0; e < E; ++e) v[e] = v[e] + p.cross_gain * (((1.0f + pg[e]) * av[e]) * inverse);
            if (blockIdx.x == 0)
#pragma unroll
                for (int e = 0; e < E; ++e) p.x_out[lane * E + e] = v[e];
            wave_lds_sync();  // the runs are read before the next squares replace them
        }
        float peak = 0.0f;
        if constexpr (NORM) {
            const float inverse = norm_inverse(v, gv, &peak);
#pragma unroll
            for (int e = 0; e < E; ++e) v[e] = v[e] * inverse;
            if (p.hidden_out != nullptr && blockIdx.x == 0)
#pragma unroll
                for (int e = 0; e < E; ++e) p.hidden_out[lane * E + e] = v[e];
            peak = peak * inverse;
        } else {
#pragma unroll
            for (int e = 0; e < E; ++e) peak = fmaxf(peak, fabsf(v[e]));
            peak = wave_max_nonneg(peak);
        }
        sx = int8_scale_from_peak(peak);
        float y[E];
        quotients<E>(v, sx, y);
#pragma unroll
        for (int e = 0; e < E; ++e) xq_s[lane * E + e] = (int8_t)code_of_quotient(y[e]);
        wave_lds_sync();
#pragma unroll
        for (int j = 0; j < NL; ++j) xc[j] = *reinterpret_cast<const int4*>(xq_s + load_chunk(j) * 16);
    }

    // 3. exact int32 group accumulators
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        int part = dot16(w[j], xc[j], 0);
        part = part + lane_xor_i<1>(part);  // the lane pair of a chunk (DPP)
        if ((lane & 1) == 0) acc_s[load_row(j) * G + load_chunk(j) / 2] = part;
    }
    wave_lds_sync();

    // 4. sequential per-row epilogue (tree T4), one lane per row
    float total = 0.0f;
    if (mine) {
        const int4* arow = reinterpret_cast<const int4*>(acc_s + lane * G);
#pragma unroll
        for (int i = 0; i < G / 4; ++i) {
            const int4 a4 = arow[i];
            const float a[4] = {(float)a4.x, (float)a4.y, (float)a4.z, (float)a4.w};
            const float s[4] = {sv[i].x, sv[i].y, sv[i].z, sv[i].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if constexpr (FORM == kPanel)
                    total = fmaf(a[k], s[k] * sx, total);  // panel.rs:184-188
                else
                    total = total + (a[k] * s[k]) * sx;    // neon.rs:180
            }
        }
    }
    if (sg.acc != nullptr)
        for (int idx = lane; idx < ROWS * G; idx += 64)
            if (row_valid(idx / G)) sg.acc[(size_t)row_of(idx / G) * G + (idx % G)] = acc_s[idx];

    if constexpr (EPI == kStore) {
        if (mine) sg.y[row_of(lane)] = total;
    } else if constexpr (EPI == kResidual) {
        if (mine) sg.y[row_of(lane)] = residual_in + total;
    } else if constexpr (EPI == kSilu) {
        const float up = lane_xor<H>(total);  // lane + H for the lanes below H (DPP / lane swap)
        if (lane < H && mine) sg.y[blk * H + lane] = silu(total) * up;
    } else {  // kArgmax: logits plus this block's greedy key (generator.rs:257-265);
              // argmax_finalize reduces the keys (device atomics would serialise)
        if (mine) sg.y[row_of(lane)] = total;
        uint64_t key = mine ? argmax_key(total, (uint32_t)row_of(lane)) : 0ull;
        key = wave_max_u64(key);
        if (lane == 0) p.keys[blockIdx.x] = (unsigned long long)key;
        // the last kernel of a greedy step (no other block reads the state)
        if (p.advance != nullptr && blockIdx.x == 0 && lane == 0) {
            p.advance->pos = p.advance->pos + 1;
            p.advance->step = p.advance->step + 1;
        }
    }
}

// The wide decode product (down, K 2048): four waves split the columns, so
// each wave quantises and dots a quarter of the input (K / 256 values a lane)
// instead of one wave doing the whole row; the per-row scale needs the peak
// of all four quarters (one exchange through LDS). A lane owns one 16-code
// chunk of one row per load; lane pairs join a 32-code group by DPP; the
// group sums meet in LDS and lane r of wave 0 runs row r's sequential
// epilogue over all K / 32 groups (tree T4), then the residual add.
template <int K, int ROWS, int FORM>
__global__ __launch_bounds__(256) void gemv_splitk_kernel(GemvParams p) {
    constexpr int W = 4;                  // waves
    constexpr int KW = K / W;             // columns per wave
    constexpr int G = K / kGroup;         // groups per row
    constexpr int GW = KW / kGroup;       // groups per row and wave
    constexpr int CW = KW / 16;           // 16-code chunks per row and wave
    constexpr int NL = ROWS * CW / 64;    // loads per lane
    constexpr int E = KW / 64;            // input values per lane
    static_assert((ROWS * CW) % 64 == 0 && E % 4 == 0 && G % 4 == 0, "whole loads, float4 inputs, scale quads");
    static_assert(ROWS <= 64, "one lane per row in the epilogue");
    __shared__ __align__(16) int8_t xq_s[K];
    __shared__ __align__(16) int acc_s[ROWS * G];
    __shared__ float peak_s[W];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const Segment sg = p.seg[0];
    const int r0 = (int)blockIdx.x * ROWS;
    // load j of a lane: chunk (64 j + lane) % CW of row (64 j + lane) / CW, in this wave's columns
    auto load_row = [&](int j) -> int { return (64 * j + lane) / CW; };
    auto load_chunk = [&](int j) -> int { return (64 * j + lane) % CW; };

    float v[E];
    load_floats<E>(p.x + wave * KW + lane * E, v);
    int4 w[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j)
        w[j] = *reinterpret_cast<const int4*>(sg.W + (size_t)min(r0 + load_row(j), sg.rows - 1) * K + wave * KW +
                                              load_chunk(j) * 16);
    const bool mine = wave == 0 && lane < ROWS && r0 + lane < sg.rows;
    float4 sv[G / 4];
    float residual_in = 0.0f;  // the row's current value, requested with the other loads
    {
        const int rr = min(r0 + min(lane, ROWS - 1), sg.rows - 1);
        const float4* src = reinterpret_cast<const float4*>(sg.sW + (size_t)rr * G);
        if (wave == 0) {
#pragma unroll
            for (int i = 0; i < G / 4; ++i) sv[i] = src[i];
            residual_in = p.res != nullptr ? p.res[rr] : sg.y[rr];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // the row scale from the peak of all four quarters (ops.rs:103-118)
    float peak = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) peak = fmaxf(peak, fabsf(v[e]));
    peak = wave_max_nonneg(peak);
    if (lane == 0) peak_s[wave] = peak;
    lds_barrier();
    peak = fmaxf(fmaxf(peak_s[0], peak_s[1]), fmaxf(peak_s[2], peak_s[3]));
    const float sx = int8_scale_from_peak(peak);
    float y[E];
    quotients<E>(v, sx, y);
#pragma unroll
    for (int e = 0; e < E; ++e) xq_s[wave * KW + lane * E + e] = (int8_t)code_of_quotient(y[e]);
    // the codes a lane dots were written by lanes of its own wave
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int4 xc = *reinterpret_cast<const int4*>(xq_s + wave * KW + load_chunk(j) * 16);
        int part = dot16(w[j], xc, 0);
        part = part + dpp_move<0xb1>(part);  // lane ^ 1 holds the other half of the group
        if ((lane & 1) == 0) acc_s[load_row(j) * G + wave * GW + load_chunk(j) / 2] = part;
    }
    lds_barrier();
    if (mine) {
        const int4* arow = reinterpret_cast<const int4*>(acc_s + lane * G);
        float total = 0.0f;
#pragma unroll
        for (int i = 0; i < G / 4; ++i) {
            const int4 a4 = arow[i];
            const float a[4] = {(float)a4.x, (float)a4.y, (float)a4.z, (float)a4.w};
            const float s[4] = {sv[i].x, sv[i].y, sv[i].z, sv[i].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if constexpr (FORM == kPanel)
                    total = fmaf(a[k], s[k] * sx, total);  // panel.rs:184-188
                else
                    total = total + (a[k] * s[k]) * sx;    // neon.rs:180
            }
        }
        sg.y[r0 + lane] = residual_in + total;
    }
}

hipError_t launch_gemv_splitk(const GemvParams& p, int columns, int rows, hipStream_t stream) {
    if (columns == 2048) {
        rn_launch((gemv_splitk_kernel<2048, 2, kPanel>), dim3((rows + 1) / 2), dim3(256), 0, stream, p);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

__global__ __launch_bounds__(256) void argmax_finalize_kernel(const unsigned long long* keys, int nkeys,
                                                              const float* logits, DecodeState* st, uint32_t* ids,
                                                              int mode) {
    __shared__ unsigned long long best_s[4];
    // rounds of four keys a thread, all requested before any compare, from
    // clamped indices (a repeated key does not change the maximum)
    uint64_t key = 0ull;
    for (int base = 0; base < nkeys; base += 4 * 256) {
        uint64_t kk[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) kk[j] = keys[min(base + (int)threadIdx.x + 256 * j, nkeys - 1)];
#pragma unroll
        for (int j = 0; j < 4; ++j) key = kk[j] > key ? kk[j] : key;
    }
    key = wave_max_u64(key);
    if ((threadIdx.x & 63) == 0) best_s[threadIdx.x >> 6] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t k = best_s[0];
        for (int w = 1; w < 4; ++w) k = best_s[w] > k ? best_s[w] : k;
        const float first = logits[0];
        const uint32_t index = (first != first) ? 0u : argmax_index(k);  // a NaN at 0 is never displaced
        st->token = index;
        const uint32_t step = st->step;
        if (mode == 0) {
            if (ids != nullptr && step < st->ids_capacity) ids[step] = index;
            st->step = step + 1;
            st->pos = st->pos + 1;
        } else if (ids != nullptr && step > 0 && step - 1 < st->ids_capacity) {
            ids[step - 1] = index;
        }
    }
}

hipError_t launch_argmax_finalize(const unsigned long long* keys, int nkeys, const float* logits,
                                  DecodeState* state, uint32_t* ids, hipStream_t stream, int mode) {
    rn_launch(argmax_finalize_kernel, dim3(1), dim3(256), 0, stream, keys, nkeys, logits, state, ids, mode);
    return hipGetLastError();
}

__global__ void greedy_start_kernel(DecodeState* st, uint32_t token, int32_t pos, uint32_t ids_capacity,
                                    unsigned long long* keys, int nkeys, float* logits) {
    for (int i = threadIdx.x; i < nkeys; i += blockDim.x) keys[i] = argmax_key(0.0f, token);
    if (threadIdx.x == 0) {
        st->token = token;
        st->pos = pos;
        st->step = 0;
        st->ids_capacity = ids_capacity;
        logits[0] = 0.0f;
    }
}

hipError_t launch_greedy_start(DecodeState* state, uint32_t token, int32_t pos, uint32_t ids_capacity,
                               unsigned long long* keys, int nkeys, float* logits, hipStream_t stream) {
    rn_launch(greedy_start_kernel, dim3(1), dim3(256), 0, stream, state, token, pos, ids_capacity, keys, nkeys,
              logits);
    return hipGetLastError();
}

template <int K, int ROWS, int PRO, int EPI, int FORM>
static hipError_t launch_one(const GemvParams& p, int blocks, hipStream_t stream) {
    rn_launch((gemv_kernel<K, ROWS, PRO, EPI, FORM>), dim3(blocks, p.nseg), dim3(64), 0, stream, p);
    return hipGetLastError();
}

template <int K, int ROWS>
static hipError_t dispatch_pe(const GemvParams& p, int prologue, int epilogue, int form, int blocks,
                              hipStream_t s) {
    // API products: quantise + store, either form.
    if (prologue == kQuant && epilogue == kStore)
        return form == kPanel ? launch_one<K, ROWS, kQuant, kStore, kPanel>(p, blocks, s)
                              : launch_one<K, ROWS, kQuant, kStore, kPlane>(p, blocks, s);
    if (prologue == kCodes && epilogue == kStore)
        return form == kPanel ? launch_one<K, ROWS, kCodes, kStore, kPanel>(p, blocks, s)
                              : launch_one<K, ROWS, kCodes, kStore, kPlane>(p, blocks, s);
    if (form == kPanel) {
        if (prologue == kQuant && epilogue == kResidual) return launch_one<K, ROWS, kQuant, kResidual, kPanel>(p, blocks, s);
        if constexpr (K == 512 || K == 384) {
            if (prologue == kClassSum && epilogue == kStore) return launch_one<K, ROWS, kClassSum, kStore, kPanel>(p, blocks, s);
            if (prologue == kNorm && epilogue == kStore) return launch_one<K, ROWS, kNorm, kStore, kPanel>(p, blocks, s);
            if (prologue == kEmbedNorm && epilogue == kStore) return launch_one<K, ROWS, kEmbedNorm, kStore, kPanel>(p, blocks, s);
            if (prologue == kNorm && epilogue == kSilu) return launch_one<K, ROWS, kNorm, kSilu, kPanel>(p, blocks, s);
            if (prologue == kCrossNorm && epilogue == kSilu) return launch_one<K, ROWS, kCrossNorm, kSilu, kPanel>(p, blocks, s);
        }
    } else {
        if constexpr (K == 512 || K == 384)
            if (prologue == kNorm && epilogue == kArgmax) return launch_one<K, ROWS, kNorm, kArgmax, kPlane>(p, blocks, s);
    }
    return hipErrorInvalidValue;
}

int gemv_rows_per_block(int rows, int columns, int epilogue) {
    if (epilogue == kSilu) return 8;
    // rows x 16-byte chunks must fill whole 64-lane loads: 384 columns need
    // multiples of 8 rows, 1536 multiples of 2
    int r, min_rows;
    switch (columns) {
        case 384: r = 32; min_rows = 8; break;
        case 512: r = 32; min_rows = 2; break;
        case 1024: r = 16; min_rows = 1; break;
        case 1536: r = 8; min_rows = 2; break;
        default: r = 8; min_rows = 1; break;
    }
    // Tall products: more rows per block amortise the input prologue, while
    // keeping >= 2048 blocks (eight waves per CU) in flight.
    while (r > 8 && (rows + r - 1) / r < 2048) r /= 2;
    // Decode-sized products: enough blocks to cover all 256 CUs.
    while (r > min_rows && (rows + r - 1) / r < 256) r /= 2;
    return r;
}

hipError_t launch_gemv(const GemvParams& p, int columns, int prologue, int epilogue, int form, int rows_per_block,
                       int blocks, hipStream_t stream) {
    if (blocks <= 0) return hipSuccess;
    switch (columns) {
        case 384:
            if (rows_per_block == 8) return dispatch_pe<384, 8>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 16) return dispatch_pe<384, 16>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 32) return dispatch_pe<384, 32>(p, prologue, epilogue, form, blocks, stream);
            break;
        case 1536:
            if (rows_per_block == 2) return dispatch_pe<1536, 2>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 4) return dispatch_pe<1536, 4>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 8) return dispatch_pe<1536, 8>(p, prologue, epilogue, form, blocks, stream);
            break;
        case 512:
            if (rows_per_block == 2) return dispatch_pe<512, 2>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 4) return dispatch_pe<512, 4>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 8) return dispatch_pe<512, 8>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 16) return dispatch_pe<512, 16>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 32) return dispatch_pe<512, 32>(p, prologue, epilogue, form, blocks, stream);
            break;
        case 1024:
            if (rows_per_block == 1) return dispatch_pe<1024, 1>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 2) return dispatch_pe<1024, 2>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 4) return dispatch_pe<1024, 4>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 8) return dispatch_pe<1024, 8>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 16) return dispatch_pe<1024, 16>(p, prologue, epilogue, form, blocks, stream);
            break;
        case 2048:
            if (rows_per_block == 1) return dispatch_pe<2048, 1>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 2) return dispatch_pe<2048, 2>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 4) return dispatch_pe<2048, 4>(p, prologue, epilogue, form, blocks, stream);
            if (rows_per_block == 8) return dispatch_pe<2048, 8>(p, prologue, epilogue, form, blocks, stream);
            break;
        default:
            break;
    }
    return hipErrorInvalidValue;
}

}  // namespace rn
