// rn_gemm.hip — multi-token quantised products on gfx950 i8 MFMA, plus the
// row kernels of batched prefill / multi-sequence decode.
//
// Replaces QuantisedMatrix::multiply_batch / multiply_natural_fused
// (crates/kernels/src/matrix.rs:277-389) and the panel tile
// (crates/kernels/src/panel.rs:136-198) for int8 codes with one fp32 scale per
// 32 columns.
//
// One v_mfma_i32_16x16x32_i8 covers exactly one 32-column group for a
// 16-token x 16-row tile, so every group's int32 sums come out of the matrix
// core separately and feed the sequential group epilogue of the reference
// (panel form fmaf(acc, sW*sx, total), or plane form total + (acc*sW)*sx).
// MFMA operand layout (16x16x32 i8): lane l supplies A row l%16 and B column
// l%16 with 8 bytes of K from quarter l/16; any K permutation inside the
// instruction is the same for A and B, so the group sum is exact regardless.
// Output register i of lane l holds row 4*(l/16) + i, column l%16.
#include "rn_device.hpp"
#include "rn_internal.hpp"

namespace rn {

// The integer work of a BM x BN output tile is spread over the 16 waves of a
// 1024-thread block by group — every (16x16 sub-tile, group) MFMA is one job, each
// wave issues all the loads of its 4 jobs at once — and the int32 group sums go
// to LDS. Then one lane per output runs the sequential epilogue chain over the
// groups, reading the sums and the weight scales from LDS. All of a tile's
// loads are in flight together, so a launch costs about one memory round trip
// plus the chain, whatever K is. LDS: G*BM*BN int32 (64 KB at the sizes used).
template <int G, int BM, int BN>
struct SplitShape {
    static constexpr int kSub = (BM / 16) * (BN / 16);  // 16x16 sub-tiles
    static constexpr int kJobs = kSub * G;
    static constexpr int kPerWave = kJobs / 16;
    static_assert(kJobs % 16 == 0, "jobs spread evenly over 16 waves");
    static_assert(G % kPerWave == 0, "a wave's jobs stay in one sub-tile");
    static_assert(BM * BN <= 1024, "one output per thread");
};

// Token rows of the split kernel: int8 codes and scales given (kRowsCodes), or
// float rows quantised in the prologue (kRowsQuant: quantise_int8 of
// ops.rs:103-118, identical to norm_quantise_kernel without gains). One wave
// per row: lane l holds elements E l .. E l + E - 1. kRowsNormQuant: the same
// after the zero-centred norm with `gain` (identical to norm_quantise_kernel
// with gains; 16-row tiles, one row per wave).
enum RowsIn { kRowsCodes = 0, kRowsQuant = 1, kRowsNormQuant = 2 };

template <int G, int BM, int BN, int EPI, int FORM, bool DUMP, int AIN>
__global__ __launch_bounds__(1024) void gemm_split_kernel(GemmParams p) {
    using S = SplitShape<G, BM, BN>;
    constexpr bool kSilu = EPI == kGemmSilu;
    constexpr int K = G * kGroup;
    static_assert(AIN == kRowsCodes || (BM % 16 == 0 && K % 64 == 0), "whole rows per wave, whole elements per lane");
    static_assert(AIN != kRowsNormQuant || BM == 16, "one normed row per wave");
    // Operand rows padded by 32 bytes: the 16 rows x 4 quarters of one MFMA
    // fragment read then cover all 64 banks twice (the minimum for 512 bytes).
    constexpr int KP = K + 32;
    constexpr int kOperandBytes = (BM + BN) * KP;
    constexpr int kAccBytes = G * BM * BN * 4;
    // operand tiles first, then (after every wave has its fragments) the sums
    __shared__ __align__(16) char ops_s[kOperandBytes > kAccBytes ? kOperandBytes : kAccBytes];
    int8_t(*a_s)[KP] = reinterpret_cast<int8_t(*)[KP]>(ops_s);
    int8_t(*b_s)[KP] = reinterpret_cast<int8_t(*)[KP]>(ops_s + BM * KP);
    int(*acc_s)[BM][BN] = reinterpret_cast<int(*)[BM][BN]>(ops_s);
    __shared__ float sw_s[BN][G + 1];
    __shared__ float sx_s[BM];
    __shared__ float tile[kSilu ? BM : 1][kSilu ? BN + 1 : 1];
    // kRowsNormQuant: a wave's squares, run r (elements e = r mod 8) at r * (K / 8 + 4)
    __shared__ __align__(16) float sq_s[AIN == kRowsNormQuant ? 16 : 1][AIN == kRowsNormQuant ? K + 32 : 1];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int mtiles = (p.M + BM - 1) / BM;
    int t = blockIdx.x;
    if ((gridDim.x & 7) == 0) t = (t & 7) * (gridDim.x >> 3) + (t >> 3);
    const int mt = t % mtiles, nt = t / mtiles;
    const int m0 = mt * BM;

    // float token rows (kRowsQuant): requested first, wave w owns rows w,
    // w + 16, ...; rows past the matrix repeat its last row
    constexpr int E = AIN != kRowsCodes ? K / 64 : 1;
    constexpr int RPW = AIN != kRowsCodes ? BM / 16 : 1;
    float xv[RPW][E];
    if constexpr (AIN != kRowsCodes) {
#pragma unroll
        for (int rr = 0; rr < RPW; ++rr)
            load_floats<E>(p.Xf + (size_t)min(m0 + wave + 16 * rr, p.M - 1) * K + lane * E, xv[rr]);
    }
    // the norm gains, requested with the rows (not after them: that load
    // would then start only when the rows had arrived)
    float gv[AIN == kRowsNormQuant ? E : 1];
    if constexpr (AIN == kRowsNormQuant) load_floats<E>(p.gain + lane * E, gv);

    // output column of local column c (silu: first BN/2 gate rows, then the up rows)
    auto column = [&](int c) -> int {
        if constexpr (kSilu)
            return c < BN / 2 ? nt * (BN / 2) + c : p.half + nt * (BN / 2) + (c - BN / 2);
        else
            return nt * BN + c;
    };

    // phase 1a: the tile's token rows and weight rows into LDS with 16-byte
    // loads (a 64-lane load covers 1 KB of consecutive row bytes), all issued
    // before any is waited for; rows past the matrix repeat its last row
    constexpr int kRow16 = K / 16;  // 16-byte pieces per row
    constexpr int kFirst = AIN != kRowsCodes ? BM * kRow16 : 0;  // float rows: weight pieces only
    constexpr int kPieces = (BM + BN) * kRow16 - kFirst;
    v4i piece[(kPieces + 1023) / 1024];  // native vectors stay in registers
#pragma unroll
    for (int q = 0; q < (kPieces + 1023) / 1024; ++q) {
        const int i = kFirst + threadIdx.x + 1024 * q;
        if (kPieces % 1024 == 0 || i < kFirst + kPieces) {
            const int row = i / kRow16, col = i - row * kRow16;
            const int8_t* src = row < BM ? p.X + (size_t)min(m0 + row, p.M - 1) * K
                                         : p.W + (size_t)min(column(row - BM), p.N - 1) * K;
            piece[q] = *reinterpret_cast<const v4i*>(src + 16 * col);
        }
    }
    // scales of the tile's columns (into registers; stored to LDS after the
    // token rows are quantised, so that no wave waits for them before that)
    constexpr int kScaleLoads = (BN * G + 1023) / 1024;
    float swv[kScaleLoads];
#pragma unroll
    for (int q = 0; q < kScaleLoads; ++q) {
        const int i = min((int)threadIdx.x + 1024 * q, BN * G - 1), c = i / G, g = i - c * G;
        swv[q] = p.sW[(size_t)min(column(c), p.N - 1) * G + g];
    }
    if (AIN == kRowsCodes && threadIdx.x < BM) sx_s[threadIdx.x] = p.sx[min(m0 + (int)threadIdx.x, p.M - 1)];
    // the residual add's current value of this thread's output, requested now
    // rather than after the group chain (each output belongs to one thread)
    float residual_in = 0.0f;
    if constexpr (EPI == kGemmResidual) {
        const int rr = min((int)threadIdx.x / BN, BM - 1), cc = (int)threadIdx.x - ((int)threadIdx.x / BN) * BN;
        residual_in = p.Y[(size_t)min(m0 + rr, p.M - 1) * p.ldy + min(column(cc), p.N - 1)];
    }
    // the operand pieces and scales into LDS: for float token rows after their
    // quantisation below (which waits only for the rows), else now
    auto store_pieces = [&]() {
#pragma unroll
        for (int q = 0; q < (kPieces + 1023) / 1024; ++q) {
            const int i = kFirst + threadIdx.x + 1024 * q;
            if (kPieces % 1024 == 0 || i < kFirst + kPieces) {
                const int row = i / kRow16, col = i - row * kRow16;
                *reinterpret_cast<v4i*>(&a_s[0][0] + (size_t)row * KP + 16 * col) = piece[q];
            }
        }
#pragma unroll
        for (int q = 0; q < kScaleLoads; ++q) {
            const int i = (int)threadIdx.x + 1024 * q;
            if (i < BN * G) sw_s[i / G][i % G] = swv[q];
        }
    };
    if constexpr (AIN == kRowsCodes) store_pieces();
    if constexpr (AIN != kRowsCodes) {
        // the token rows' codes and scales, one wave per row
#pragma unroll
        for (int rr = 0; rr < RPW; ++rr) {
            const int row = wave + 16 * rr;
            float* v = xv[rr];
            float peak = 0.0f;
            if constexpr (AIN == kRowsNormQuant) {
                // the ordered 8-run sum of squares of norm_quantise_kernel (ops.rs:7-17),
                // the gained values m = (1 + g) x and their peak beside it; the normed
                // peak is fl(peak(|m|) * inverse) (rounding is monotone, inverse > 0)
                // (runs padded by four floats: 16-byte reads, and the eight
                // summing lanes start on banks 4 apart)
                constexpr int run = K / 8, stride = run + 4;
                float* sq = sq_s[wave];
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const int ge = lane * E + e;
                    sq[(ge & 7) * stride + (ge >> 3)] = v[e] * v[e];
                }
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    v[e] = (1.0f + gv[e]) * v[e];
                    peak = fmaxf(peak, fabsf(v[e]));
                }
                peak = wave_max_nonneg(peak);
                // a wave's own squares: DS operations of a wave complete in order
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                float part = 0.0f;
                if (lane < 8) {
                    const float4* r = reinterpret_cast<const float4*>(sq + lane * stride);
#pragma unroll
                    for (int c = 0; c < run / 4; ++c) {
                        const float4 t = r[c];
                        part = part + t.x;
                        part = part + t.y;
                        part = part + t.z;
                        part = part + t.w;
                    }
                }
                float total = sum_lanes_0_to_7(part);
                total = total + 0.0f;  // the empty tail of the 8-lane sum
                const float inverse = reciprocal(sqrtf(total / (float)K + p.eps));
#pragma unroll
                for (int e = 0; e < E; ++e) v[e] = v[e] * inverse;
                peak = peak * inverse;
            } else {
#pragma unroll
                for (int e = 0; e < E; ++e) peak = fmaxf(peak, fabsf(v[e]));
                peak = wave_max_nonneg(peak);
            }
            const float scale = int8_scale_from_peak(peak);
            float y[E];
            quotients<E>(v, scale, y);
            int8_t* dst = &a_s[row][lane * E];
#pragma unroll
            for (int e = 0; e < E; e += 2) {
                const uint32_t lo = (uint32_t)(uint8_t)(int8_t)code_of_quotient(y[e]);
                const uint32_t hi = (uint32_t)(uint8_t)(int8_t)code_of_quotient(y[e + 1]);
                *reinterpret_cast<uint16_t*>(dst + e) = (uint16_t)(lo | (hi << 8));
            }
            if (lane == 0) sx_s[row] = scale;
        }
        store_pieces();
    }
    __syncthreads();

    // phase 1b: this wave's jobs — one sub-tile, kPerWave consecutive groups
    const int job0 = wave * S::kPerWave;
    const int sub = job0 / G, g0 = job0 - sub * G;
    const int sm = (sub / (BN / 16)) * 16, sn = (sub % (BN / 16)) * 16;
    const int r16 = lane & 15, kq = lane >> 4;
    long a[S::kPerWave], b[S::kPerWave];
#pragma unroll
    for (int q = 0; q < S::kPerWave; ++q) {
        a[q] = *reinterpret_cast<const long*>(&a_s[sm + r16][(g0 + q) * kGroup + 8 * kq]);
        b[q] = *reinterpret_cast<const long*>(&b_s[sn + r16][(g0 + q) * kGroup + 8 * kq]);
    }
    v4i r4[S::kPerWave];
#pragma unroll
    for (int q = 0; q < S::kPerWave; ++q)
        r4[q] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[q], b[q], v4i{0, 0, 0, 0}, 0, 0, 0);
    __syncthreads();  // every wave holds its fragments: the operand tiles may be overwritten
#pragma unroll
    for (int q = 0; q < S::kPerWave; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc_s[g0 + q][sm + 4 * kq + i][sn + r16] = r4[q][i];
    __syncthreads();

    // phase 2: one output per thread, the group chain in order
    const int r = threadIdx.x / BN, c = threadIdx.x - r * BN;
    float total = 0.0f;
    if (r < BM) {
        const float sx = sx_s[r];
#pragma unroll 8
        for (int g = 0; g < G; ++g) {
            const int v = acc_s[g][r][c];
            const float s = sw_s[c][g];
            if constexpr (FORM == kPanel)
                total = fmaf((float)v, s * sx, total);  // panel.rs:184-188
            else
                total = total + ((float)v * s) * sx;    // neon.rs:180
        }
        if constexpr (DUMP) {
            const int m = m0 + r, n = column(c);
            if (m < p.M && n < p.N)
                for (int g = 0; g < G; ++g) p.acc[((size_t)m * p.N + n) * G + g] = acc_s[g][r][c];
        }
    }
    if constexpr (kSilu) {
        if (r < BM) tile[r][c] = total;
        __syncthreads();
        if (threadIdx.x < BM * (BN / 2)) {
            const int mi = threadIdx.x / (BN / 2), ii = threadIdx.x - mi * (BN / 2);
            const int m = m0 + mi, o = nt * (BN / 2) + ii;
            if (m < p.M && o < p.half) p.Y[(size_t)m * p.ldy + o] = silu(tile[mi][ii]) * tile[mi][BN / 2 + ii];
        }
    } else if (r < BM) {
        const int m = m0 + r, n = column(c);
        if (m < p.M && n < p.N) {
            float* dst = p.Y + (size_t)m * p.ldy + n;
            if constexpr (EPI == kGemmResidual)
                *dst = residual_in + total;
            else if constexpr (EPI == kGemmStoreSilu)
                *dst = silu(total);  // stem.rs:76,99: silu after the stage
            else
                *dst = total;
        }
    }
}

// ---- the chain GEMM: group chains kept in the MFMA result registers ----------
//
// A 256-thread block (4 waves, WAVES_M x (4 / WAVES_M)) owns a BM x BN output
// tile; each wave owns SM x SN sub-tiles of 16 x 16, and each lane 4 outputs per
// sub-tile (rows 4 (l / 16) .. +3, column l % 16). For every 32-column group the
// wave issues one v_mfma_i32_16x16x32_i8 per sub-tile and folds the int32 group
// sum straight into the lane's running totals in group order (panel form
// fmaf(acc, sW * sx, total), plane form total + (acc * sW) * sx), so no sum
// leaves the registers. K streams through LDS in chunks of 4 groups (128 bytes
// of every tile row), double-buffered: the next chunk's operand pieces and
// weight scales are requested before the current chunk's MFMAs, and written to
// the other buffer after them; one barrier per chunk. For the gated FFN
// (SN = 2) sub-tile column 0 holds gate rows and column 1 the matching up rows,
// so silu(gate) * up needs no exchange.
constexpr int kChunkGroups = 4;                  // groups per K chunk
constexpr int kChunkBytes = kChunkGroups * kGroup;  // 128
constexpr int kChunkPitch = kChunkBytes + 16;    // LDS row pitch: 16-byte aligned, rows start on different banks

template <int SM, int SN, int WAVES_M, int EPI, int FORM, bool DUMP>
__global__ __launch_bounds__(256) void gemm_chain_kernel(GemmParams p) {
    constexpr int WAVES_N = 4 / WAVES_M;
    constexpr int BM = WAVES_M * SM * 16, BN = WAVES_N * SN * 16;
    constexpr bool kSilu = EPI == kGemmSilu;
    static_assert(!kSilu || SN == 2, "the gated FFN pairs gate and up sub-tiles");
    constexpr int kPieces = (BM + BN) * (kChunkBytes / 16);  // 16-byte pieces per chunk
    constexpr int kPer = (kPieces + 255) / 256;
    __shared__ __align__(16) int8_t a_s[2][BM][kChunkPitch];
    __shared__ __align__(16) int8_t b_s[2][BN][kChunkPitch];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int mtiles = (p.M + BM - 1) / BM;
    int t = blockIdx.x;
    if ((gridDim.x & 7) == 0) t = (t & 7) * (gridDim.x >> 3) + (t >> 3);  // one weight panel per XCD
    const int mt = t % mtiles, nt = t / mtiles;
    const int m0 = mt * BM;
    const int G = p.K / kGroup, chunks = G / kChunkGroups;

    // weight row of local tile column c (silu: wave column block wn holds 16
    // outputs; its sub-tile column 0 is their gate rows, column 1 their up rows)
    auto weight_row = [&](int c) -> int {
        if constexpr (kSilu) {
            const int w = c / 32, j = (c / 16) & 1, o = nt * (BN / 2) + w * 16 + (c & 15);
            return j == 0 ? o : p.half + o;
        } else {
            return nt * BN + c;
        }
    };
    auto row_ok = [&](int c) -> bool {
        if constexpr (kSilu) return nt * (BN / 2) + (c / 32) * 16 + (c & 15) < p.half;
        else return nt * BN + c < p.N;
    };

    // the chunk's operand pieces: piece i is 16-byte column i % 8 of tile row
    // i / 8 (rows 0..BM-1 tokens, then BN weight rows); rows past the matrix
    // repeat its last row
    v4i piece[kPer];
    auto load_chunk = [&](int ch) {
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int i = min((int)threadIdx.x + 256 * q, kPieces - 1);
            const int row = i >> 3, col = i & 7;
            const int8_t* src = row < BM ? p.X + (size_t)min(m0 + row, p.M - 1) * p.K
                                         : p.W + (size_t)min(weight_row(row - BM), p.N - 1) * p.K;
            piece[q] = *reinterpret_cast<const v4i*>(src + (size_t)ch * kChunkBytes + 16 * col);
        }
    };
    auto store_chunk = [&](int buf) {
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int i = (int)threadIdx.x + 256 * q;
            if (kPieces % 256 == 0 || i < kPieces) {
                const int row = i >> 3, col = i & 7;
                int8_t* dst = row < BM ? &a_s[buf][row][16 * col] : &b_s[buf][row - BM][16 * col];
                *reinterpret_cast<v4i*>(dst) = piece[q];
            }
        }
    };
    // this lane's weight rows (one per sub-tile column) and token rows
    const int r16 = lane & 15, kq = lane >> 4;
    int wrow[SN];
#pragma unroll
    for (int j = 0; j < SN; ++j) wrow[j] = min(weight_row(wn * SN * 16 + j * 16 + r16), p.N - 1);
    float4 sw[SN];
    auto load_scales = [&](int ch) {
#pragma unroll
        for (int j = 0; j < SN; ++j)
            sw[j] = *reinterpret_cast<const float4*>(p.sW + (size_t)wrow[j] * G + ch * kChunkGroups);
    };
    float sx[SM][4];
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) sx[i][r] = p.sx[min(m0 + wm * SM * 16 + i * 16 + 4 * kq + r, p.M - 1)];

    float total[SM][SN][4];
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) total[i][j][r] = 0.0f;

    load_chunk(0);
    load_scales(0);
    store_chunk(0);
    __syncthreads();
    for (int ch = 0; ch < chunks; ++ch) {
        const int buf = ch & 1;
        float4 swc[SN];
#pragma unroll
        for (int j = 0; j < SN; ++j) swc[j] = sw[j];
        if (ch + 1 < chunks) {
            load_chunk(ch + 1);
            load_scales(ch + 1);
        }
#pragma unroll
        for (int gk = 0; gk < kChunkGroups; ++gk) {
            long a[SM], b[SN];
#pragma unroll
            for (int i = 0; i < SM; ++i)
                a[i] = *reinterpret_cast<const long*>(&a_s[buf][wm * SM * 16 + i * 16 + r16][gk * kGroup + 8 * kq]);
#pragma unroll
            for (int j = 0; j < SN; ++j)
                b[j] = *reinterpret_cast<const long*>(&b_s[buf][wn * SN * 16 + j * 16 + r16][gk * kGroup + 8 * kq]);
#pragma unroll
            for (int i = 0; i < SM; ++i)
#pragma unroll
                for (int j = 0; j < SN; ++j) {
                    const v4i acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[i], b[j], v4i{0, 0, 0, 0}, 0, 0, 0);
                    const float s = gk == 0 ? swc[j].x : gk == 1 ? swc[j].y : gk == 2 ? swc[j].z : swc[j].w;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if constexpr (FORM == kPanel)
                            total[i][j][r] = fmaf((float)acc[r], s * sx[i][r], total[i][j][r]);  // panel.rs:184-188
                        else
                            total[i][j][r] = total[i][j][r] + ((float)acc[r] * s) * sx[i][r];  // neon.rs:180
                    }
                    if constexpr (DUMP) {
                        const int n = nt * BN + wn * SN * 16 + j * 16 + r16;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int m = m0 + wm * SM * 16 + i * 16 + 4 * kq + r;
                            if (m < p.M && n < p.N)
                                p.acc[((size_t)m * p.N + n) * G + ch * kChunkGroups + gk] = acc[r];
                        }
                    }
                }
        }
        if (ch + 1 < chunks) {
            store_chunk(buf ^ 1);
            __syncthreads();
        }
    }

    // epilogue
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + wm * SM * 16 + i * 16 + 4 * kq + r;
            if (m >= p.M) continue;
            if constexpr (kSilu) {
                const int o = nt * (BN / 2) + wn * 16 + r16;
                if (o < p.half) p.Y[(size_t)m * p.ldy + o] = silu(total[i][0][r]) * total[i][1][r];
            } else {
#pragma unroll
                for (int j = 0; j < SN; ++j) {
                    const int c = wn * SN * 16 + j * 16 + r16;
                    if (!row_ok(c)) continue;
                    float* dst = p.Y + (size_t)m * p.ldy + nt * BN + c;
                    if constexpr (EPI == kGemmResidual)
                        *dst = *dst + total[i][j][r];
                    else if constexpr (EPI == kGemmStoreSilu)
                        *dst = silu(total[i][j][r]);  // stem.rs:76,99: silu after the stage
                    else
                        *dst = total[i][j][r];
                }
            }
        }
}

// ---- the panel GEMM: the tile's whole K panel in LDS ----------------------------
//
// The chain kernel's arithmetic (a 16 x 16 x 32 i8 MFMA per sub-tile and group,
// folded into the lane's running totals in group order), with every operand
// byte of the block requested at once: the tile's weight scales, then the BM
// token rows and BN weight rows in K chunks of 128 columns (four groups),
// chunk by chunk, go straight to LDS (global_load_lds_dwordx4, no registers).
// Every wave issues the same number of chunk loads, so the group chains of
// chunk c start once the wave's loads of chunks 0..c are in (a counted vmcnt
// wait, then an LDS barrier) while the later chunks are still arriving. A
// chunk's rows are 128 bytes, their eight 16-byte pieces XOR-swizzled by the
// row (piece p of row r at slot p ^ (r & 7)), so the rows of an MFMA fragment
// read spread over the banks without padding.
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void global_void;

template <int K, int BM, int BN>
struct PanelShape {
    static constexpr int kChunks = K / 128;               // K chunks of 128 columns
    static constexpr int kChunkBytes = (BM + BN) * 128;    // a chunk's LDS image
    static constexpr int kChunkRounds = kChunkBytes / 16 / 256;  // loads a wave issues per chunk
    static constexpr int kG = K / kGroup;
    static constexpr int kScaleSlots = BN * kG / 4;   // 16-byte pieces of the tile's weight scales
    static_assert(K % 128 == 0 && (BM + BN) % 32 == 0, "whole chunks, whole load rounds");
};

template <int K, int SM, int SN, int WAVES_M, int EPI, int FORM>
__global__ __launch_bounds__(256) void gemm_panel_kernel(GemmParams p) {
    constexpr int WAVES_N = 4 / WAVES_M;
    constexpr int BM = WAVES_M * SM * 16, BN = WAVES_N * SN * 16;
    using S = PanelShape<K, BM, BN>;
    constexpr int G = S::kG;
    constexpr bool kSilu = EPI == kGemmSilu;
    constexpr bool kRope = EPI == kGemmRope;
    static_assert(!kSilu || SN == 2, "the gated FFN pairs gate and up sub-tiles");
    static_assert(!kRope || (SM == 1 && SN == 1 && WAVES_M == 2), "rotary: wave column 0 the first halves, 1 the second");
    static_assert(K % 32 == 0 && G % 4 == 0, "whole groups, scale quads");
    // one array a chunk, so that the reads of a chunk are seen not to alias the
    // later chunks' loads into LDS (which the compiler would otherwise wait for)
    __shared__ __align__(16) int8_t chunk0_s[S::kChunkBytes], chunk1_s[S::kChunkBytes], chunk2_s[S::kChunkBytes];
    __shared__ __align__(16) int8_t chunk3_s[S::kChunks > 3 ? S::kChunkBytes : 16];
    static_assert(S::kChunks >= 3 && S::kChunks <= 4, "K of 384 or 512");
    auto chunk_s = [&](int ch) -> int8_t* { return ch == 0 ? chunk0_s : ch == 1 ? chunk1_s : ch == 2 ? chunk2_s : chunk3_s; };
    __shared__ __align__(16) float sw_s[BN * G];
    __shared__ float pair_s[kRope ? BM : 1][kRope ? BN + 1 : 1];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int mtiles = (p.M + BM - 1) / BM;
    int t = blockIdx.x;
    if ((gridDim.x & 7) == 0) t = (t & 7) * (gridDim.x >> 3) + (t >> 3);  // one weight panel per XCD
    const int mt = t % mtiles, nt = t / mtiles;
    const int m0 = mt * BM;

    // weight row of local tile column c (silu: wave column block wn holds 16
    // outputs; its sub-tile column 0 is their gate rows, column 1 their up rows;
    // rotary: tiles nt = 2 hp + s cover pairs 16 s .. 16 s + 15 of head row
    // block hp, wave column 0 their first halves, wave column 1 their second)
    auto weight_row = [&](int c) -> int {
        if constexpr (kSilu) {
            const int w = c / 32, j = (c / 16) & 1, o = nt * (BN / 2) + w * 16 + (c & 15);
            return j == 0 ? o : p.half + o;
        } else if constexpr (kRope) {
            return (nt >> 1) * 64 + (c >> 4) * 32 + (nt & 1) * 16 + (c & 15);
        } else {
            return nt * BN + c;
        }
    };
    auto row_ok = [&](int c) -> bool {
        if constexpr (kSilu) return nt * (BN / 2) + (c / 32) * 16 + (c & 15) < p.half;
        else if constexpr (kRope) return (nt >> 1) * 64 < p.N;
        else return nt * BN + c < p.N;
    };

    const int r16 = lane & 15, kq = lane >> 4;
    // the rows' activation scales (register loads, issued before the panel's
    // loads so that the counted waits below cover them)
    float sx[SM][4];
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) sx[i][r] = p.sx[min(m0 + wm * SM * 16 + i * 16 + 4 * kq + r, p.M - 1)];
    // 1. the tile's weight scales, then the panel chunk by chunk: slot s of
    // chunk c's image (tile row s / 8, rows 0..BM-1 tokens, then BN weight
    // rows; rows past the matrix repeat its last row) holds 16-byte piece
    // (s % 8) ^ (row & 7) of the row's columns 128 c .. 128 c + 127. A wave's
    // lanes fill 64 consecutive slots per load.
#pragma unroll
    for (int q = 0; q < (S::kScaleSlots + 255) / 256; ++q) {
        const int sl = 256 * q + 64 * wave + lane;
        if (sl < S::kScaleSlots) {
            const int c = sl / (G / 4), quad = sl - c * (G / 4);
            __builtin_amdgcn_global_load_lds((global_void*)(p.sW + (size_t)min(weight_row(c), p.N - 1) * G + 4 * quad),
                                             (lds_void*)(sw_s + 4 * (256 * q + 64 * wave)), 16, 0, 0);
        }
    }
#pragma unroll
    for (int ch = 0; ch < S::kChunks; ++ch)
#pragma unroll
        for (int q = 0; q < S::kChunkRounds; ++q) {
            const int sl = 256 * q + 64 * wave + lane, row = sl >> 3, piece = (sl & 7) ^ (row & 7);
            const int8_t* src = row < BM ? p.X + (size_t)min(m0 + row, p.M - 1) * K
                                         : p.W + (size_t)min(weight_row(row - BM), p.N - 1) * K;
            __builtin_amdgcn_global_load_lds((global_void*)(src + 128 * ch + 16 * piece),
                                             (lds_void*)(chunk_s(ch) + 16 * (256 * q + 64 * wave)),
                                             16, 0, 0);
        }
    float total[SM][SN][4];
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) total[i][j][r] = 0.0f;

    // 2. the group chains, in group order, a chunk at a time. Lane (r16, kq)
    // reads bytes 8 kq .. 8 kq + 7 of a group of fragment row r16: piece
    // 2 (g % 4) + kq / 2 of the chunk row, half kq % 2.
    int arow[SM], brow[SN];
    const float* srow[SN];
#pragma unroll
    for (int i = 0; i < SM; ++i) arow[i] = (wm * SM * 16 + i * 16 + r16) * 128 + 8 * (kq & 1);
#pragma unroll
    for (int j = 0; j < SN; ++j) {
        brow[j] = (BM + wn * SN * 16 + j * 16 + r16) * 128 + 8 * (kq & 1);
        srow[j] = sw_s + (wn * SN * 16 + j * 16 + r16) * G;
    }
    int slot[4];
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) slot[gg] = ((2 * gg + (kq >> 1)) ^ (r16 & 7)) * 16;
#pragma unroll
    for (int ch = 0; ch < S::kChunks; ++ch) {
        // this wave's loads of chunks 0..ch are in (later chunks' loads, the
        // newest, may still be outstanding); then every wave's
        constexpr int kRounds = S::kChunkRounds;
        switch (S::kChunks - 1 - ch) {
            case 0: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
            case 1: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRounds)); break;
            case 2: __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * kRounds)); break;
            default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(3 * kRounds)); break;
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const int8_t* chunk = chunk_s(ch);
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
            const int g = 4 * ch + gg;
            long a[SM], b[SN];
            float sv[SN];
#pragma unroll
            for (int i = 0; i < SM; ++i) a[i] = *reinterpret_cast<const long*>(chunk + arow[i] + slot[gg]);
#pragma unroll
            for (int j = 0; j < SN; ++j) {
                b[j] = *reinterpret_cast<const long*>(chunk + brow[j] + slot[gg]);
                sv[j] = srow[j][g];
            }
#pragma unroll
            for (int i = 0; i < SM; ++i)
#pragma unroll
                for (int j = 0; j < SN; ++j) {
                    const v4i acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[i], b[j], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if constexpr (FORM == kPanel)
                            total[i][j][r] = fmaf((float)acc[r], sv[j] * sx[i][r], total[i][j][r]);  // panel.rs:184-188
                        else
                            total[i][j][r] = total[i][j][r] + ((float)acc[r] * sv[j]) * sx[i][r];  // neon.rs:180
                    }
                }
        }
    }

    // 3. epilogue
    if constexpr (kRope) {
        // the rotate-half pairs (i, i + 32) of one head meet in LDS; then a
        // thread per (row, pair) as rope_append_kernel does for one token
#pragma unroll
        for (int r = 0; r < 4; ++r) pair_s[wm * 16 + 4 * kq + r][wn * 16 + r16] = total[0][0][r];
        __syncthreads();
        const int hp = nt >> 1, part = hp / p.rope.heads, h = hp - part * p.rope.heads;
        const int d = p.rope.heads * 64;
#pragma unroll
        for (int e = tid; e < BM * 16; e += 256) {
            const int lr = e >> 4, pi = e & 15, m = m0 + lr;
            if (m >= p.M || part > 2) continue;
            const int i = (nt & 1) * 16 + pi, pos = p.rope.first + m;
            const float a = pair_s[lr][pi], b = pair_s[lr][16 + pi];
            const size_t base = (((size_t)p.rope.layer * p.rope.heads + h) * p.rope.capacity + pos) * 64;
            if (part == 2) {
                p.rope.vc[base + i] = __float2half_rn(a);
                p.rope.vc[base + i + 32] = __float2half_rn(b);
            } else {
                const float c = p.rope.cos[(size_t)pos * 32 + i], s = p.rope.sin[(size_t)pos * 32 + i];
                const float x0 = a * c - b * s, x1 = b * c + a * s;
                if (part == 0) {
                    p.rope.q_out[(size_t)m * d + h * 64 + i] = x0;
                    p.rope.q_out[(size_t)m * d + h * 64 + i + 32] = x1;
                } else {
                    p.rope.kc[base + i] = __float2half_rn(x0);
                    p.rope.kc[base + i + 32] = __float2half_rn(x1);
                }
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + wm * SM * 16 + i * 16 + 4 * kq + r;
            if (m >= p.M) continue;
            if constexpr (kSilu) {
                const int o = nt * (BN / 2) + wn * 16 + r16;
                if (o < p.half) p.Y[(size_t)m * p.ldy + o] = silu(total[i][0][r]) * total[i][1][r];
            } else {
#pragma unroll
                for (int j = 0; j < SN; ++j) {
                    const int c = wn * SN * 16 + j * 16 + r16;
                    if (!row_ok(c)) continue;
                    float* dst = p.Y + (size_t)m * p.ldy + nt * BN + c;
                    if constexpr (EPI == kGemmResidual)
                        *dst = *dst + total[i][j][r];
                    else if constexpr (EPI == kGemmStoreSilu)
                        *dst = silu(total[i][j][r]);  // stem.rs:76,99: silu after the stage
                    else
                        *dst = total[i][j][r];
                }
            }
        }
}

template <int SM, int SN, int WAVES_M, int EPI, int FORM, bool DUMP>
static void launch_chain(const GemmParams& p, hipStream_t stream) {
    constexpr int BM = WAVES_M * SM * 16, BN = (4 / WAVES_M) * SN * 16;
    const int mtiles = (p.M + BM - 1) / BM;
    const int ntiles = EPI == kGemmSilu ? (p.half + BN / 2 - 1) / (BN / 2) : (p.N + BN - 1) / BN;
    const dim3 grid(mtiles * ntiles), block(256);
    if constexpr (!DUMP) {
        // the whole K panel in LDS for the widths it fits
        switch (p.K) {
            case 384: rn_launch((gemm_panel_kernel<384, SM, SN, WAVES_M, EPI, FORM>), grid, block, 0, stream, p); return;
            case 512: rn_launch((gemm_panel_kernel<512, SM, SN, WAVES_M, EPI, FORM>), grid, block, 0, stream, p); return;
            default: break;
        }
    }
    if constexpr (EPI != kGemmRope) rn_launch((gemm_chain_kernel<SM, SN, WAVES_M, EPI, FORM, DUMP>), grid, block, 0, stream, p);
}

// Tile shape: the one with the most blocks among 64 x 64, 64 x 32, 32 x 64 and
// 32 x 32 (not for the gated FFN, whose waves pair gate and up sub-tiles). The
// chains are VALU-bound, so blocks (waves) are the parallelism: small tiles
// measured faster than large ones at every size used here, also with the
// panel's loads overlapping the chains (64 x 64 re-reads less but ran the
// 256-token gate/up product slower than 64 x 32).
// Returns the chain shape to use (0-3), or -1 for the split kernel.
template <int EPI>
static int chain_pick(const GemmParams& p) {
    const int n_eff = EPI == kGemmSilu ? 2 * p.half : p.N;
    auto blocks = [&](int bm, int bn) { return ((p.M + bm - 1) / bm) * ((n_eff + bn - 1) / bn); };
    struct Shape { int bm, bn; };
    const Shape shapes[4] = {{64, 64}, {64, 32}, {32, 64}, {32, 32}};
    const int count = EPI == kGemmSilu ? 3 : 4;
    int pick = -1, best = 0;
    for (int i = 0; i < count; ++i) {
        const int b = blocks(shapes[i].bm, shapes[i].bn);
        if (b > best) { best = b; pick = i; }
    }
    // Under 256 blocks the per-block chain over K is the critical path and the
    // split kernel (all groups of a tile in flight at once) is faster.
    return best < 256 ? -1 : pick;
}

template <int EPI, int FORM, bool DUMP>
static void launch_chain_shape(const GemmParams& p, int pick, hipStream_t stream) {
    switch (pick) {
        case 0: launch_chain<2, 2, 2, EPI, FORM, DUMP>(p, stream); break;
        case 1: launch_chain<1, 2, 4, EPI, FORM, DUMP>(p, stream); break;
        case 2: launch_chain<1, 2, 2, EPI, FORM, DUMP>(p, stream); break;
        default:
            if constexpr (EPI != kGemmSilu) launch_chain<1, 1, 2, EPI, FORM, DUMP>(p, stream);
            break;
    }
}

template <int G, int BM, int BN, int EPI, int FORM, bool DUMP, int AIN>
static void launch_split(const GemmParams& p, hipStream_t stream) {
    const int mtiles = (p.M + BM - 1) / BM;
    const int ntiles = EPI == kGemmSilu ? (p.half + BN / 2 - 1) / (BN / 2) : (p.N + BN - 1) / BN;
    rn_launch((gemm_split_kernel<G, BM, BN, EPI, FORM, DUMP, AIN>), dim3(mtiles * ntiles), dim3(1024), 0, stream, p);
}

// 16-row tiles where the 16 waves divide the jobs: these grids are small, and
// at 512 columns twice the blocks of 32-row tiles measured faster at 64 and
// 256 rows (16 x 16 tiles did not)
template <int EPI, int FORM, bool DUMP, int AIN>
static void launch_by_rows(const GemmParams& p, hipStream_t stream) {
    switch (p.K) {
        case 384:
            launch_split<12, 32, 32, EPI, FORM, DUMP, AIN>(p, stream);
            break;
        case 512:
            launch_split<16, 16, 32, EPI, FORM, DUMP, AIN>(p, stream);
            break;
        case 1024:
            launch_split<32, 16, 32, EPI, FORM, DUMP, AIN>(p, stream);
            break;
        case 1536:
            launch_split<48, 16, 16, EPI, FORM, DUMP, AIN>(p, stream);
            break;
        default:
            launch_split<64, 16, 16, EPI, FORM, DUMP, AIN>(p, stream);
            break;
    }
}

// The chain kernel for large grids, the split kernel for small ones. Float
// input rows without a norm are quantised inside the split kernel when that
// re-reads little: every column tile of the grid quantises its own rows
// again, so the fused form is taken for rows of at most 512 and at most 8 MB of
// re-read floats per launch (measured: the batch-64 and 256-token out products
// gain about 1.8 us; wider or taller grids do not). Float rows of 512 with a
// norm are normed and quantised in the prologue up to 16 MB of re-read at
// 32-column tiles, on 64-column tiles above 8 MB (the batch-64 QKV product: 6.9
// us against 4.5 + 3.8 us for the product and the norm launch; its gate/up
// product on 64-column tiles: 0.90 -> 0.88 ms per step, where 32-column tiles
// measured a loss). Otherwise a quantise launch (with the norm when `gain` is
// set) writes the codes to X / sx first.
template <int EPI, int FORM, bool DUMP, int AIN>
static hipError_t launch_product(const GemmParams& p, hipStream_t stream) {
    if constexpr (EPI == kGemmRope) {
        // the 32 x 32 panel tile at every size (its epilogue pairs the two wave columns)
        if (AIN != kRowsCodes) {
            const hipError_t e = launch_norm_quantise(p.Xf, p.gain, p.M, p.K, p.eps, const_cast<int8_t*>(p.X),
                                                      const_cast<float*>(p.sx), nullptr, stream);
            if (e != hipSuccess) return e;
        }
        launch_chain<1, 1, 2, kGemmRope, FORM, false>(p, stream);
        return hipGetLastError();
    } else {
    const int pick = p.K == 1152 ? (EPI == kGemmSilu ? 2 : 3) : chain_pick<EPI>(p);
    const int n_eff = EPI == kGemmSilu ? 2 * p.half : p.N;
    const size_t reread = (size_t)((n_eff + 31) / 32) * (size_t)p.M * (size_t)p.K * sizeof(float);
    const bool fused =
        AIN != kRowsCodes && p.gain == nullptr && pick < 0 && p.K <= 512 && reread <= ((size_t)8 << 20);
    const bool fused_norm =
        AIN != kRowsCodes && p.gain != nullptr && pick < 0 && p.K == 512 && reread <= ((size_t)16 << 20);
    if (AIN != kRowsCodes && !fused && !fused_norm) {
        const hipError_t e = launch_norm_quantise(p.Xf, p.gain, p.M, p.K, p.eps, const_cast<int8_t*>(p.X),
                                                  const_cast<float*>(p.sx), nullptr, stream);
        if (e != hipSuccess) return e;
    }
    if (pick >= 0)
        launch_chain_shape<EPI, FORM, DUMP>(p, pick, stream);
    else if (fused)
        launch_by_rows<EPI, FORM, DUMP, kRowsQuant>(p, stream);
    else if (fused_norm && reread <= ((size_t)8 << 20))
        launch_split<16, 16, 32, EPI, FORM, DUMP, kRowsNormQuant>(p, stream);
    else if (fused_norm)  // 64-column tiles: half the re-read of 32-column tiles
        launch_split<16, 16, 64, EPI, FORM, DUMP, kRowsNormQuant>(p, stream);
    else
        launch_by_rows<EPI, FORM, DUMP, kRowsCodes>(p, stream);
    return hipGetLastError();
    }
}

template <int EPI>
static hipError_t launch_panel(const GemmParams& p, int ain, hipStream_t stream) {
    return ain == kRowsQuant ? launch_product<EPI, kPanel, false, kRowsQuant>(p, stream)
                             : launch_product<EPI, kPanel, false, kRowsCodes>(p, stream);
}

hipError_t launch_gemm(const GemmParams& p, int epilogue, int form, bool dump, hipStream_t stream) {
    if (p.M <= 0) return hipSuccess;
    // instantiated for the supported widths (the kernel is unrolled over groups)
    if ((p.K != 384 && p.K != 512 && p.K != 1024 && p.K != 1152 && p.K != 1536 && p.K != 2048) || p.N <= 0)
        return hipErrorInvalidValue;
    // 1152 columns (the stem's im2col rows at d 384) have no split-kernel tile: codes only, chain kernel
    if (p.K == 1152 && (p.Xf != nullptr || dump)) return hipErrorInvalidValue;
    if (epilogue == kGemmSilu && (p.half % 16 != 0 || p.N != 2 * p.half)) return hipErrorInvalidValue;
    if (epilogue == kGemmRope &&
        (dump || form != kPanel || (p.K != 384 && p.K != 512) || p.rope.heads <= 0 || p.N != 3 * 64 * p.rope.heads ||
         p.rope.q_out == nullptr || p.rope.kc == nullptr || p.rope.vc == nullptr || p.rope.cos == nullptr ||
         p.rope.sin == nullptr || p.rope.first < 0 || p.rope.first + p.M > p.rope.capacity))
        return hipErrorInvalidValue;
    if (p.Xf != nullptr && (p.X == nullptr || p.sx == nullptr)) return hipErrorInvalidValue;
    const int ain = p.Xf == nullptr ? kRowsCodes : kRowsQuant;
    if (dump || form == kPlane) {
        // the dump and plane-form products take codes: float rows are quantised first
        if (epilogue != kGemmStore) return hipErrorInvalidValue;
        if (ain != kRowsCodes) {
            const hipError_t e = launch_norm_quantise(p.Xf, p.gain, p.M, p.K, p.eps, const_cast<int8_t*>(p.X),
                                                      const_cast<float*>(p.sx), nullptr, stream);
            if (e != hipSuccess) return e;
        }
        if (dump)
            return form == kPanel ? launch_product<kGemmStore, kPanel, true, kRowsCodes>(p, stream)
                                  : launch_product<kGemmStore, kPlane, true, kRowsCodes>(p, stream);
        return launch_product<kGemmStore, kPlane, false, kRowsCodes>(p, stream);
    }
    switch (epilogue) {
        case kGemmStore: return launch_panel<kGemmStore>(p, ain, stream);
        case kGemmResidual: return launch_panel<kGemmResidual>(p, ain, stream);
        case kGemmSilu: return launch_panel<kGemmSilu>(p, ain, stream);
        case kGemmStoreSilu: return launch_panel<kGemmStoreSilu>(p, ain, stream);
        case kGemmRope: return launch_panel<kGemmRope>(p, ain, stream);
        default: return hipErrorInvalidValue;
    }
}

// ---- row kernels for multi-token work -------------------------------------------

// Optional zero-centred norm (ops.rs:44-50 with the sum of ops.rs:7-17), then
// the per-row int8 quantisation (ops.rs:112-118). One wave per row, four rows
// per block; the row lives in registers (n/128 float2 per lane). The sum of
// squares keeps the reference's order: 8 strided partial sums (element e goes
// to partial e%8, each summed in element order), then the partials 0..7 in
// order; the squares are staged transposed in LDS so that each of 8 lanes runs
// one partial over contiguous memory. `normed` (nullable) receives the normed
// rows. NV = n / 128 float2 per lane.
template <int NV>
__global__ __launch_bounds__(256) void norm_quantise_kernel(const float* x, const float* gain, int count, float eps,
                                                            int8_t* codes, float* scales, float* normed,
                                                            size_t x_stride) {
    constexpr int n = NV * 128;
    extern __shared__ float sq_s[];  // [waves][n + 32] when gain != nullptr
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + wave;
    const bool live = row < count;
    const float2* src = reinterpret_cast<const float2*>(x + (size_t)(live ? row : count - 1) * x_stride);
    float2 v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = src[lane + 64 * i];
    float peak = 0.0f;
    if (gain != nullptr) {
        // run r of the squares at sq[r * (run + 4)]: 16-byte aligned runs whose
        // 128-bit reads by the 8 chain lanes fall in distinct banks
        constexpr int run = n >> 3, stride = run + 4;
        float* sq = sq_s + wave * (n + 32);
        const float2* g2 = reinterpret_cast<const float2*>(gain);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int e = 2 * (lane + 64 * i);  // elements e, e+1; e % 8 is 0, 2, 4 or 6
            const int p = e & 7, c = e >> 3;
            sq[(p + 0) * stride + c] = v[i].x * v[i].x;
            sq[(p + 1) * stride + c] = v[i].y * v[i].y;
        }
        // the gained values and their peak while the squares are summed: the
        // normed value is fl(m * inverse) with inverse > 0 and rounding is
        // monotone, so the normed peak is fl(peak(|m|) * inverse)
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const float2 g = g2[lane + 64 * i];
            v[i].x = (1.0f + g.x) * v[i].x;
            v[i].y = (1.0f + g.y) * v[i].y;
            peak = fmaxf(peak, fmaxf(fabsf(v[i].x), fabsf(v[i].y)));
        }
        peak = wave_max_nonneg(peak);
        wave_lds_sync();  // each wave reads only its own row's squares
        float part = 0.0f;
        if (lane < 8) {
            // the run in 128-bit reads, each group of CH requested before its adds
            constexpr int R4 = run / 4, CH = R4 % 16 == 0 ? 16 : (R4 % 12 == 0 ? 12 : 4);
            static_assert(R4 % CH == 0, "whole groups of reads");
            const float4* r4 = reinterpret_cast<const float4*>(sq + lane * stride);
#pragma unroll
            for (int c0 = 0; c0 < R4; c0 += CH) {
                float4 t[CH];
#pragma unroll
                for (int c = 0; c < CH; ++c) t[c] = r4[c0 + c];
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    part = part + t[c].x;
                    part = part + t[c].y;
                    part = part + t[c].z;
                    part = part + t[c].w;
                }
            }
        }
        float total = sum_lanes_0_to_7(part);
        total = total + 0.0f;  // the empty tail of the 8-lane sum
        const float inverse = reciprocal(sqrtf(total / (float)n + eps));
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            v[i].x = v[i].x * inverse;
            v[i].y = v[i].y * inverse;
            if (normed != nullptr && live) reinterpret_cast<float2*>(normed + (size_t)row * n)[lane + 64 * i] = v[i];
        }
        peak = peak * inverse;
    } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) peak = fmaxf(peak, fmaxf(fabsf(v[i].x), fabsf(v[i].y)));
        peak = wave_max_nonneg(peak);
    }
    const float scale = int8_scale_from_peak(peak);
    if (!live) return;  // the whole wave: one row per wave
    if (codes != nullptr) {
        float y[2 * NV];
        quotients<2 * NV>(reinterpret_cast<const float*>(v), scale, y);
        uint16_t* dst = reinterpret_cast<uint16_t*>(codes + (size_t)row * n);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t b0 = (uint8_t)code_of_quotient(y[2 * i + 0]);
            const uint32_t b1 = (uint8_t)code_of_quotient(y[2 * i + 1]);
            dst[lane + 64 * i] = (uint16_t)(b0 | (b1 << 8));
        }
    }
    if (lane == 0 && scales != nullptr) scales[row] = scale;
}

hipError_t launch_norm_quantise(const float* x, const float* gain, int count, int n, float eps, int8_t* codes,
                                float* scales, float* normed, hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    // one row a block: the rows' loads spread over as many CUs as there are rows
    const size_t lds = gain != nullptr ? sizeof(float) * (size_t)(n + 32) : 0;
    const dim3 grid(count), block(64);
#define RN_NQ(NV) \
    rn_launch(norm_quantise_kernel<NV>, grid, block, lds, stream, x, gain, count, eps, codes, scales, normed, (size_t)n)
    switch (n) {
        case 384: RN_NQ(3); break;
        case 512: RN_NQ(4); break;
        case 1024: RN_NQ(8); break;
        case 1152: RN_NQ(9); break;
        case 1536: RN_NQ(12); break;
        case 2048: RN_NQ(16); break;
        default: return hipErrorInvalidValue;
    }
#undef RN_NQ
    return hipGetLastError();
}

hipError_t launch_quantise_strided(const float* x, size_t x_stride, int count, int n, int8_t* codes, float* scales,
                                   hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    const dim3 grid(count), block(64);
    const float* no_gain = nullptr;
    float* no_normed = nullptr;
#define RN_QS(NV) \
    rn_launch(norm_quantise_kernel<NV>, grid, block, 0, stream, x, no_gain, count, 0.0f, codes, scales, no_normed, x_stride)
    switch (n) {
        case 1152: RN_QS(9); break;
        case 1536: RN_QS(12); break;
        default: return hipErrorInvalidValue;
    }
#undef RN_QS
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
// One 1024-thread block a row; 16-byte loads, four in flight a thread, when
// the row allows them.
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const float* logits, int n, uint32_t* tokens, uint32_t* ids,
                                                           int steps, int step, const int32_t* step_dev) {
    __shared__ unsigned long long best_s[16];
    const float* row = logits + (size_t)blockIdx.x * n;
    const int tid = threadIdx.x;
    uint64_t key = 0ull;
    auto take = [&](float v, int i) {
        const uint64_t k = argmax_key(v, (uint32_t)i);
        key = k > key ? k : key;
    };
    if ((n & 3) == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0) {
        const float4* r4 = reinterpret_cast<const float4*>(row);
        const int n4 = n / 4;
        int i = tid;
        for (; i + 3 * 1024 < n4; i += 4 * 1024) {
            float4 v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = r4[i + j * 1024];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = 4 * (i + j * 1024);
                take(v[j].x, e);
                take(v[j].y, e + 1);
                take(v[j].z, e + 2);
                take(v[j].w, e + 3);
            }
        }
        for (; i < n4; i += 1024) {
            const float4 v = r4[i];
            take(v.x, 4 * i);
            take(v.y, 4 * i + 1);
            take(v.z, 4 * i + 2);
            take(v.w, 4 * i + 3);
        }
    } else {
        for (int i = tid; i < n; i += 1024) take(row[i], i);
    }
    key = wave_max_u64(key);
    if ((tid & 63) == 0) best_s[tid >> 6] = key;
    __syncthreads();
    if (tid == 0) {
        uint64_t k = best_s[0];
        for (int w = 1; w < 16; ++w) k = best_s[w] > k ? best_s[w] : k;
        const float first = row[0];
        const uint32_t index = (first != first) ? 0u : argmax_index(k);
        tokens[blockIdx.x] = index;
        const int at = step_dev != nullptr ? *step_dev : step;
        if (ids != nullptr && at >= 0 && at < steps) ids[(size_t)blockIdx.x * steps + at] = index;
    }
}

hipError_t launch_argmax_rows(const float* logits, int count, int n, uint32_t* tokens, uint32_t* ids, int steps,
                              int step, hipStream_t stream, const int32_t* step_dev) {
    if (count <= 0) return hipSuccess;
    rn_launch(argmax_rows_kernel, dim3(count), dim3(1024), 0, stream, logits, n, tokens, ids, steps, step, step_dev);
    return hipGetLastError();
}

__global__ void advance_positions_kernel(int32_t* pos, int count, int by, int32_t* step) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) pos[i] = pos[i] + by;
    if (step != nullptr && i == 0) *step = *step + 1;
}

hipError_t launch_advance_positions(int32_t* pos, int count, int by, hipStream_t stream, int32_t* step) {
    if (count <= 0) return hipSuccess;
    rn_launch(advance_positions_kernel, dim3((count + 255) / 256), dim3(256), 0, stream, pos, count, by, step);
    return hipGetLastError();
}

}  // namespace rn
