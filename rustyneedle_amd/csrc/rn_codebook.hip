// rn_codebook.hip — products over the codebook weight format for gfx950.
//
// A codebook-quantised [rows][columns] matrix (docs/format.md "Codebook-quantised
// matrices", cact record.rs:57-84) pads columns to a multiple of the group
// size. Its blob holds the packed indices, least-significant bits first, then
// one fp16 L2 norm per (row, group). The device keeps that blob as the
// archive stores it (2 or 4 bits a weight, 4-8x fewer bytes than int8 codes).
//
// Replaces, for the integer path the reference takes on aarch64:
//   walsh::rotate_groups (walsh.rs:41-80) under QuantisedMatrix::prepare
//     (matrix.rs:123-138)                                   -> cb_rotate_kernel
//   plane_input / NaturalInput::new per-group input codes (matrix.rs:205-214,
//     neon.rs:63-106, panel.rs:52-66), PanelMatrix::tile (panel.rs:153-197,
//     2-bit) and row_dot_two_bit / row_dot_four_bit (neon.rs:126-183, 4-bit
//     and ternary crumbs)                                    -> cb_product_kernel
//   QuantisedMatrix::dequantise_row (matrix.rs:140-153)      -> cb_dequantise_kernel
//
// Product arithmetic (bit-exact with the reference order):
//   - per group of the rotated input: scale = peak / 127 (1.0 for a zero
//     peak), code = round-half-even(x / scale) (clamped to +-127; |x| <= peak
//     keeps every quotient within +-127.5, so no clamp is reached);
//   - the integer levels (IntegerLevels, neon.rs:114-124: an int8 table and
//     one scale lscale, computed on the host) decode each index with
//     v_perm_b32 from a table held in registers, and v_dot4_i32_i8 adds the
//     exact int32 group sum (order-free);
//   - per row, sequentially over the groups:
//       2-bit (panel.rs:184-188):   total = fmaf(acc, (norm * lscale) * xs, total)
//       4-bit and ternary (neon.rs:158,180):
//                                   total = total + (((acc * norm) * lscale) * xs)
//
// Input codes live in LDS in "plane" order so that one decoded weight dword
// meets one code dword: for 2-bit indices, a dword of 16 indices holds element
// 4b + k at bits 2k of byte b, so (dword >> 2k) & 0x03030303 selects elements
// {k, 4+k, 8+k, 12+k}; the codes of each run of 16 elements are stored as the
// 4x4 byte transpose. For 4-bit indices a dword holds 8 elements and
// (dword >> 4k) & 0x0f0f0f0f selects {k, 2+k, 4+k, 6+k}.
#include "rn_device.hpp"
#include "rn_internal.hpp"

namespace rn {

namespace {

// The Walsh-Hadamard transform of one group held as runs of 16 consecutive
// elements, one run per lane, GROUP / 16 aligned lanes per group (walsh.rs:41-76):
// butterflies of span 1, 2, 4, 8 inside the lane, then spans 16 .. GROUP/2
// across lanes (partner lane ^ span/16); the low element becomes a + b, the
// high one a - b; then every value times `scale` = 1 / sqrt(GROUP).
template <int GROUP>
__device__ __forceinline__ void wht_run(float (&v)[16], int lane, float scale) {
#pragma unroll
    for (int span = 1; span < 16; span *= 2)
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if ((i & span) == 0) {
                const float a = v[i], b = v[i + span];
                v[i] = a + b;
                v[i + span] = a - b;
            }
#pragma unroll
    for (int m = 1; m < GROUP / 16; m *= 2) {
        const bool high = (lane & m) != 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float p = __shfl_xor(v[i], m, 64);
            v[i] = high ? p - v[i] : v[i] + p;
        }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = v[i] * scale;
}

// Maximum over aligned sets of L lanes (L = 1, 2, 4, 8 or 16), the same in
// every lane of the set (DPP inside rows of 16; the maximum is order-free).
template <int L>
__device__ __forceinline__ float set_max(float v) {
    if constexpr (L >= 2) v = fmaxf(v, __int_as_float(dpp_move<0xb1>(__float_as_int(v))));
    if constexpr (L >= 4) v = fmaxf(v, __int_as_float(dpp_move<0x4e>(__float_as_int(v))));
    if constexpr (L >= 8) v = fmaxf(v, __int_as_float(dpp_move<0x141>(__float_as_int(v))));
    if constexpr (L >= 16) v = fmaxf(v, __int_as_float(dpp_move<0x140>(__float_as_int(v))));
    return v;
}

// Integer sum over aligned sets of L lanes, the same in every lane of the set.
template <int L>
__device__ __forceinline__ int set_sum(int v) {
    if constexpr (L >= 2) v = v + dpp_move<0xb1>(v);
    if constexpr (L >= 4) v = v + dpp_move<0x4e>(v);
    if constexpr (L >= 8) v = v + dpp_move<0x141>(v);
    return v;
}

// The codes of one run of 16 elements in plane order for BITS-bit indices.
template <int BITS>
__device__ __forceinline__ int4 plane_pack(const int (&c)[16]) {
    auto b4 = [](int a, int b, int x, int d) -> int {
        return (a & 0xff) | ((b & 0xff) << 8) | ((x & 0xff) << 16) | ((d & 0xff) << 24);
    };
    if constexpr (BITS == 2)  // dword k = elements k, 4+k, 8+k, 12+k
        return make_int4(b4(c[0], c[4], c[8], c[12]), b4(c[1], c[5], c[9], c[13]), b4(c[2], c[6], c[10], c[14]),
                         b4(c[3], c[7], c[11], c[15]));
    else  // two blocks of 8: dword 2h + k = elements 8h + k, 8h+2+k, 8h+4+k, 8h+6+k
        return make_int4(b4(c[0], c[2], c[4], c[6]), b4(c[1], c[3], c[5], c[7]), b4(c[8], c[10], c[12], c[14]),
                         b4(c[9], c[11], c[13], c[15]));
}

// The int8 levels of four indices (one per byte of sel, 0..3 or 0..15).
template <int BITS>
__device__ __forceinline__ int decode4(uint32_t sel, const uint32_t (&lut)[4]) {
    if constexpr (BITS == 2) {
        return (int)__builtin_amdgcn_perm(0u, lut[0], sel);
    } else {
        const uint32_t s7 = sel & 0x07070707u;
        const uint32_t lo = __builtin_amdgcn_perm(lut[1], lut[0], s7);
        const uint32_t hi = __builtin_amdgcn_perm(lut[3], lut[2], s7);
        const uint32_t m = ((sel >> 3) & 0x01010101u) * 0xffu;
        return (int)((hi & m) | (lo & ~m));
    }
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) { return __half2float(__ushort_as_half(h)); }

constexpr int kNormWindow = 12288;  // bytes of norms staged per row group (3 x 16 B a thread)

}  // namespace

// QuantisedMatrix::prepare / prepare_batch (matrix.rs:123-138): x [count][columns]
// -> rotated [count][padded], zero past `columns`, each group rotated. One
// lane per run of 16 elements.
template <int GROUP>
__global__ __launch_bounds__(256) void cb_rotate_kernel(const float* x, int count, int columns, int padded,
                                                        float scale, float* rotated) {
    const int lane = threadIdx.x & 63;
    const int runs = padded / 16;
    const int f = blockIdx.x * 256 + threadIdx.x;  // flat run index over [count][runs]
    // every lane of a group set runs the shuffles, also past the end (whole
    // sets only: runs is a multiple of GROUP / 16)
    const int ff = min(f, count * runs - 1);
    const int t = ff / runs, u = ff - t * runs;
    float v[16];
    const float* src = x + (size_t)t * columns;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int e = 16 * u + i;
        v[i] = e < columns ? src[e] : 0.0f;
    }
    wht_run<GROUP>(v, lane, scale);
    if (f < count * runs) {
        float4* dst = reinterpret_cast<float4*>(rotated + (size_t)t * padded + 16 * u);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    }
}

// QuantisedMatrix::dequantise_row (matrix.rs:140-153): per group
// (level[index] * norm) then the group's Walsh-Hadamard transform; the first
// `columns` values. One block of padded / 16 lanes (at most 1024).
template <int BITS, int GROUP>
__global__ __launch_bounds__(1024) void cb_dequantise_kernel(CodebookParams p, int row, float* out) {
    constexpr int IB = BITS == 5 ? 2 : BITS;
    const int u = threadIdx.x, lane = u & 63;
    const int runs = p.padded / 16, G = p.padded / GROUP;
    const int uu = min(u, runs - 1);
    const uint8_t* r = p.packed + (size_t)row * p.row_bytes + (size_t)uu * 2 * IB;  // 16 indices = 2 * IB bytes
    const float norm = half_bits_to_float(p.norms[(size_t)row * G + (16 * uu) / GROUP]);
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int bit = i * IB;
        uint32_t raw = r[bit / 8];
        if ((bit % 8) + IB > 8) raw |= (uint32_t)r[bit / 8 + 1] << 8;  // a 3-bit index may straddle two bytes
        const int idx = (raw >> (bit % 8)) & ((1 << IB) - 1);
        v[i] = p.levels[idx] * norm;
    }
    wht_run<GROUP>(v, lane, p.wht_scale);
    if (u < runs)
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (16 * u + i < p.columns) out[16 * u + i] = v[i];
}

// The row products of T tokens at a time (token tile blockIdx.y). A block of
// four waves shares one prologue; each wave owns R = p.rows_per_block rows of a
// row group of 4R rows, and the block runs p.iters consecutive row groups so
// that a wide input is quantised once for many rows.
//   1. The first 256 runs of 16 input values are requested, then row group 0's
//      weight chunks (NL 16-byte loads a lane: chunk 64 j + lane of the wave's
//      rows in row-major order, clamped to the matrix, so no load is
//      conditional) and its norms (a 12 KB window from a 16-byte aligned
//      start; the allocation runs 16 KB past the norms).
//   2. Prologue: per run, the group's peak over its GROUP/16 lanes (DPP),
//      scale, codes (quotients without a division unless one lies near a
//      rounding boundary), stored in plane order.
//   3. Per row group: decoded dwords meet code dwords in v_dot4 and the chunks
//      of one group join across their lanes (DPP) into the wave's acc_s; the
//      next row group's loads are issued before this one's epilogue;
//   4. one lane per (token, row): the sequential group epilogue.
template <int BITS, int GROUP, int FORM, int NL, int T>
__device__ __forceinline__ void cb_product_body(const CodebookParams& p, const float* x, int count, float* y,
                                                int32_t* acc_out) {
    constexpr int IB = BITS == 5 ? 2 : BITS;        // index bits (ternary crumbs are 2)
    constexpr int EPC = 128 / IB;                    // elements per 16-byte chunk
    constexpr int CPG = GROUP / EPC;                 // chunks per group
    constexpr int RPG = GROUP / 16;                  // runs of 16 per group
    constexpr int NW = 4, NT = NW * 64;
    static_assert(CPG >= 1 && CPG <= 8 && RPG <= 16, "group of 64, 128 or 256");
    extern __shared__ __align__(16) unsigned char lds[];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int R = p.rows_per_block, CPR = p.cpr, G = p.padded / GROUP, runs = p.padded / 16;
    const int BR = NW * R, t0 = blockIdx.y * T;
    uint16_t* nm_s = reinterpret_cast<uint16_t*>(lds);                                 // 12 KB of norms
    int8_t* xq_s = reinterpret_cast<int8_t*>(lds + kNormWindow);                      // [T][padded]
    int* acc_all = reinterpret_cast<int*>(lds + kNormWindow + (size_t)T * p.padded);  // [NW][T][R][G]
    float* sx_s = reinterpret_cast<float*>(acc_all + (size_t)NW * T * R * G);         // [T][G]
    int* acc_s = acc_all + (size_t)wv * T * R * G;

    // 1. requests
    const int xruns = T * runs;  // flat (token, run) index of the tile
    auto load_run = [&](int f, float (&v)[16]) {
        const int ff = min(f, xruns - 1);
        const int t = ff / runs;
        const float4* s = reinterpret_cast<const float4*>(x + (size_t)min(t0 + t, count - 1) * p.padded +
                                                          16 * (ff - t * runs));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 q = s[i];
            v[4 * i] = q.x;
            v[4 * i + 1] = q.y;
            v[4 * i + 2] = q.z;
            v[4 * i + 3] = q.w;
        }
    };
    float xv[16];
    load_run(tid, xv);
    // With DB, row groups alternate between two sets of weight registers and a
    // group's weights are requested before the previous group's decode;
    // otherwise (wide rows, token tiles: no registers to spare) after it.
    constexpr bool DB = NL == 8 && T == 1;
    v4i wa[NL], wb[DB ? NL : 1];
    v4i nv[3];  // native vectors stay in registers (arrays of int4 structs may not)
    auto group_row0 = [&](int it) -> int { return (blockIdx.x * p.iters + it) * BR; };
    auto issue = [&](int it, auto& w) {
        const int rw = group_row0(it) + wv * R;
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int idx = 64 * j + lane;
            const int rl = (int)(((float)idx + 0.5f) * p.inv_cpr);  // exact idx / CPR for idx < 4096
            const int row = min(rw + rl, p.rows - 1);
            w[j] = *reinterpret_cast<const v4i*>(p.packed + (size_t)row * p.row_bytes + (size_t)(idx - rl * CPR) * 16);
        }
    };
    // the norms are wanted only by the epilogue: requested after the prologue,
    // so their registers are not held through it
    // (only the pieces the row group's norms cover: a full window per group
    // would fetch up to six times the norm bytes)
    auto issue_norms = [&](int it) {
        const size_t nbase = (size_t)min(group_row0(it), p.rows - 1) * G * 2, nal = nbase & ~(size_t)15;
        const int need = (int)(nbase - nal) + BR * G * 2;
#pragma unroll
        for (int i = 0; i < 3; ++i)
            if (16 * (tid + NT * i) < need)
                nv[i] = *reinterpret_cast<const v4i*>(reinterpret_cast<const unsigned char*>(p.norms) + nal +
                                                      16 * (size_t)(tid + NT * i));
    };
    issue(0, wa);
    __builtin_amdgcn_sched_barrier(0);

    // 2. prologue: per-group input codes and scales
    auto quantise_run = [&](float (&v)[16], int f) {
        float peak = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) peak = fmaxf(peak, fabsf(v[i]));
        peak = set_max<RPG>(peak);
        const float sx = int8_scale_from_peak(peak);
        // quotients four at a time: the weight loads in flight hold registers,
        // and sixteen interleaved boundary checks would add sixty more
        int c[16];
#pragma unroll
        for (int c4 = 0; c4 < 16; c4 += 4) {
            float q[4];
            quotients<4>(v + c4, sx, q);
#pragma unroll
            for (int i = 0; i < 4; ++i) c[c4 + i] = code_of_quotient(q[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (f < xruns) {
            reinterpret_cast<int4*>(xq_s)[f] = plane_pack<IB>(c);
            const int t = f / runs, u = f - t * runs;
            if (u % RPG == 0) sx_s[t * G + u / RPG] = sx;
        }
    };
    quantise_run(xv, tid);
    for (int base = NT; base < xruns; base += NT) {  // wide inputs or many tokens
        load_run(base + tid, xv);
        quantise_run(xv, base + tid);
    }

    issue_norms(0);
    const uint32_t lut[4] = {p.lut[0], p.lut[1], p.lut[2], p.lut[3]};
    // one row group: its norms to LDS, the next group's requests (into the
    // other register set, so they are in flight through this decode), the
    // group sums, the epilogue
    auto step = [&](int it, v4i (&w)[NL], auto& w_next) {
        const int gr0 = group_row0(it), rw = gr0 + wv * R;
        const int nhalf0 = (int)((((size_t)min(gr0, p.rows - 1) * G * 2) & 15) / 2);
#pragma unroll
        for (int i = 0; i < 3; ++i) reinterpret_cast<v4i*>(nm_s)[tid + NT * i] = nv[i];
        __syncthreads();  // codes, scales and this row group's norms
        if (DB && it + 1 < p.iters) issue(it + 1, w_next);

        // 3. exact int32 group sums
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int idx = 64 * j + lane;
            const int rl = (int)(((float)idx + 0.5f) * p.inv_cpr);
            const int c = idx - rl * CPR;
            int part[T];
#pragma unroll
            for (int t = 0; t < T; ++t) part[t] = 0;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t wd = (uint32_t)w[j][d];
                if constexpr (IB == 2) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int lv = decode4<2>((wd >> (2 * k)) & 0x03030303u, lut);
#pragma unroll
                        for (int t = 0; t < T; ++t) {
                            const int a =
                                *reinterpret_cast<const int*>(xq_s + (size_t)t * p.padded + 64 * c + 16 * d + 4 * k);
                            part[t] = dot4(lv, a, part[t]);
                        }
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        const int lv = decode4<4>((wd >> (4 * k)) & 0x0f0f0f0fu, lut);
#pragma unroll
                        for (int t = 0; t < T; ++t) {
                            const int a =
                                *reinterpret_cast<const int*>(xq_s + (size_t)t * p.padded + 32 * c + 8 * d + 4 * k);
                            part[t] = dot4(lv, a, part[t]);
                        }
                    }
                }
            }
            const bool store = (lane % CPG) == 0 && idx < R * CPR && rw + rl < p.rows;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int s = set_sum<CPG>(part[t]);
                if (store) acc_s[((size_t)t * R + rl) * G + c / CPG] = s;
            }
            // one chunk's code reads at a time: hoisting them all would hold
            // 16 registers a chunk and cut the waves a CU keeps in flight
            __builtin_amdgcn_sched_barrier(0);
        }
        if (it + 1 < p.iters) {  // the registers are free now
            if (!DB) issue(it + 1, w_next);
            issue_norms(it + 1);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();  // acc_s is this wave's own
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // 4. sequential epilogue per (token, row)
        for (int e = lane; e < T * R; e += 64) {
            const int t = e / R, r = e - t * R;
            if (rw + r >= p.rows || t0 + t >= count) continue;
            const int* a = acc_s + ((size_t)t * R + r) * G;
            const uint16_t* nm = nm_s + nhalf0 + (wv * R + r) * G;
            const float* xs = sx_s + t * G;
            float total = 0.0f;
            for (int g = 0; g < G; ++g) {
                const float norm = half_bits_to_float(nm[g]);
                if constexpr (FORM == kPanel)
                    total = fmaf((float)a[g], (norm * p.lscale) * xs[g], total);  // panel.rs:184-188
                else
                    total = total + ((((float)a[g] * norm) * p.lscale) * xs[g]);  // neon.rs:158,180
            }
            y[(size_t)(t0 + t) * p.rows + rw + r] = total;
            if (acc_out != nullptr)
                for (int g = 0; g < G; ++g) acc_out[((size_t)(t0 + t) * p.rows + rw + r) * G + g] = a[g];
        }
        __syncthreads();  // the norms window and acc_s are read before the next row group replaces them
    };
    if constexpr (DB) {
        for (int it = 0; it < p.iters; it += 2) {
            step(it, wa, wb);
            if (it + 1 < p.iters) step(it + 1, wb, wa);
        }
    } else {
        for (int it = 0; it < p.iters; ++it) step(it, wa, wa);
    }
}

template <int BITS, int GROUP, int FORM, int NL, int T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NL == 8 && T == 1 ? 3 : 1)))
void cb_product_kernel(CodebookParams p, const float* x, int count, float* y, int32_t* acc_out) {
    cb_product_body<BITS, GROUP, FORM, NL, T>(p, x, count, y, acc_out);
}

// Up to four products of one shape in one launch (blockIdx.z picks the job):
// matrices that share rows, width, format and group, one input vector each.
template <int BITS, int GROUP, int FORM, int NL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NL == 8 ? 3 : 1)))
void cb_product_jobs_kernel(CodebookJobs jobs) {
    const CodebookJob& j = jobs.job[blockIdx.z];
    cb_product_body<BITS, GROUP, FORM, NL, 1>(j.p, j.x, 1, j.y, nullptr);
}

namespace {

// LDS of a product block: norms window, [T][padded] codes, [4][T][R][G] sums, [T][G] scales
inline size_t product_lds(const CodebookParams& p, int T, int R) {
    const size_t G = (size_t)(p.padded / p.group);
    return kNormWindow + (size_t)T * p.padded + 4 * (4 * (size_t)T * R * G + (size_t)T * G);
}
inline int product_loads(const CodebookParams& p) { return p.cpr < 64 ? 8 : 16; }
inline int product_rows(const CodebookParams& p) { return min(64, 64 * product_loads(p) / p.cpr); }
constexpr size_t kProductMaxLds = 64 * 1024;

template <int BITS, int GROUP, int FORM, int T>
hipError_t launch_product_t(const CodebookParams& p, const float* x, int count, float* y, int32_t* acc,
                            hipStream_t stream) {
    const int nl = product_loads(p);
    CodebookParams q = p;
    q.rows_per_block = product_rows(p);
    const size_t lds = product_lds(p, T, q.rows_per_block);
    if (lds > kProductMaxLds) return hipErrorInvalidValue;
    // consecutive row groups per block (at least 4, or padded / 1024 for a wide
    // input, whose prologue then serves them all), while the grid keeps at
    // least 512 blocks; each group's loads are in flight during the previous
    // group's decode
    const int groups = (p.rows + 4 * q.rows_per_block - 1) / (4 * q.rows_per_block);
    q.iters = max(1, min(max(4, p.padded / 1024), groups / 512));
    const dim3 grid((groups + q.iters - 1) / q.iters, (count + T - 1) / T);
    if (nl == 8)
        rn_launch(cb_product_kernel<BITS, GROUP, FORM, 8, T>, grid, dim3(256), lds, stream, q, x, count, y, acc);
    else
        rn_launch(cb_product_kernel<BITS, GROUP, FORM, 16, T>, grid, dim3(256), lds, stream, q, x, count, y, acc);
    return hipGetLastError();
}

template <int BITS, int GROUP, int FORM>
hipError_t launch_product_g(const CodebookParams& p, const float* x, int count, float* y, int32_t* acc,
                            hipStream_t stream) {
    // token tiles of 8 share each block's weight loads; one token a block when
    // 8 tokens' codes would not fit the LDS budget
    const bool tile = count > 1 && product_lds(p, 8, product_rows(p)) <= kProductMaxLds;
    return tile ? launch_product_t<BITS, GROUP, FORM, 8>(p, x, count, y, acc, stream)
                : launch_product_t<BITS, GROUP, FORM, 1>(p, x, count, y, acc, stream);
}

template <int BITS, int FORM>
hipError_t launch_product_b(const CodebookParams& p, const float* x, int count, float* y, int32_t* acc,
                            hipStream_t stream) {
    switch (p.group) {
        case 64: return launch_product_g<BITS, 64, FORM>(p, x, count, y, acc, stream);
        case 128: return launch_product_g<BITS, 128, FORM>(p, x, count, y, acc, stream);
        case 256: return launch_product_g<BITS, 256, FORM>(p, x, count, y, acc, stream);
        default: return hipErrorInvalidValue;
    }
}

// ---- the float path (x86-64 and the 1- and 3-bit widths) ----------------------
//
// The level of element e of a packed row, LSB first (matrix.rs:623-631); a
// 3-bit index may straddle two bytes.
__device__ __forceinline__ float cb_level(const uint8_t* row, int e, int ib, const float* levels) {
    const int bit = e * ib, byte = bit >> 3, shift = bit & 7;
    uint32_t raw = row[byte];
    if (shift + ib > 8) raw |= (uint32_t)row[byte + 1] << 8;
    return levels[(raw >> shift) & ((1u << ib) - 1)];
}

// fill_rows_float (matrix.rs:427-440) for one token (blockIdx.y) and rb rows
// (blockIdx.x): a chain is (row, group, lane) of LookupTable::dot_group
// (matrix.rs:610-620): lane l of the N = 8 / index_bits values of a byte sums
// level * input over the group's bytes in order from 0.0; 3-bit groups are one
// chain over the positions from -0.0 (N = 1). The lanes of a group are summed
// in order from -0.0 (Iterator::sum), then one thread per row adds
// partial * norm over the groups in order from 0.0.
__global__ __launch_bounds__(256) void cb_float_vector_kernel(CodebookParams p, const float* x, float* y, int rb,
                                                              int nl) {
    extern __shared__ float sh[];  // [rb][groups][nl] lane sums, then [rb][groups] partials
    const int ib = p.bits == 5 ? 2 : p.bits, groups = p.padded / p.group;
    const int row0 = blockIdx.x * rb, token = blockIdx.y;
    const float* xt = x + (size_t)token * p.padded;
    const int per_row = groups * nl, chains = rb * per_row;
    float* lane_s = sh;
    float* part_s = sh + chains;
    for (int c = threadIdx.x; c < chains; c += blockDim.x) {
        const int r = c / per_row, rem = c - r * per_row, g = rem / nl, l = rem - g * nl;
        const uint8_t* row = p.packed + (size_t)min(row0 + r, p.rows - 1) * p.row_bytes;
        const int base = g * p.group;
        float acc = nl == 1 ? -0.0f : 0.0f;
        for (int b = 0; b < p.group / nl; ++b) {
            const int e = base + b * nl + l;
            acc = acc + cb_level(row, e, ib, p.levels) * xt[e];
        }
        lane_s[c] = acc;
    }
    __syncthreads();
    for (int q = threadIdx.x; q < rb * groups; q += blockDim.x) {
        float s = lane_s[q * nl];
        if (nl > 1) {
            s = -0.0f;
            for (int l = 0; l < nl; ++l) s = s + lane_s[q * nl + l];
        }
        part_s[q] = s;
    }
    __syncthreads();
    for (int r = threadIdx.x; r < rb; r += blockDim.x) {
        const int row = row0 + r;
        if (row >= p.rows) continue;
        float total = 0.0f;
        for (int g = 0; g < groups; ++g)
            total = total + part_s[r * groups + g] * half_bits_to_float(p.norms[(size_t)row * groups + g]);
        y[(size_t)token * p.rows + row] = total;
    }
}

// multiply_batch's float tile (matrix.rs:356-378): the expanded row
// (expand_row_scaled: level * norm per element, matrix.rs:390-399) dotted with
// the input in eight lanes over chunks of 8 from 0.0 (dot, matrix.rs:488-497),
// the lanes summed in order from -0.0. Eight threads per (token, row), one per lane.
__global__ __launch_bounds__(256) void cb_float_batch_kernel(CodebookParams p, const float* x, int count, float* y) {
    const int ib = p.bits == 5 ? 2 : p.bits, groups = p.padded / p.group;
    const int l = threadIdx.x & 7;
    const long long pair = (long long)blockIdx.x * 32 + (threadIdx.x >> 3);
    const bool live = pair < (long long)count * p.rows;
    const int token = live ? (int)(pair / p.rows) : 0, row = live ? (int)(pair % p.rows) : 0;
    const uint8_t* packed = p.packed + (size_t)row * p.row_bytes;
    const uint16_t* norms = p.norms + (size_t)row * groups;
    const float* xt = x + (size_t)token * p.padded;
    float acc = 0.0f;
    for (int c = 0; c < p.padded / 8; ++c) {
        const int e = 8 * c + l;
        const float w = cb_level(packed, e, ib, p.levels) * half_bits_to_float(norms[e / p.group]);
        acc = acc + w * xt[e];
    }
    float s = -0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) s = s + __shfl(acc, (threadIdx.x & ~7) + j, 64);
    if (live && l == 0) y[(size_t)token * p.rows + row] = s;
}

}  // namespace

hipError_t launch_codebook_float(const CodebookParams& p, const float* x, int count, float* y, bool batch,
                                 hipStream_t stream) {
    if (count < 1 || p.rows < 1 || p.padded % p.group != 0) return hipErrorInvalidValue;
    if (p.bits < 1 || p.bits > 5) return hipErrorInvalidValue;
    if (batch) {
        const long long pairs = (long long)count * p.rows;
        rn_launch(cb_float_batch_kernel, dim3((unsigned)((pairs + 31) / 32)), dim3(256), 0, stream, p, x, count, y);
    } else {
        const int ib = p.bits == 5 ? 2 : p.bits, nl = ib == 3 ? 1 : 8 / ib;
        const int per_row = (p.padded / p.group) * nl;
        const int rb = per_row >= 256 ? 1 : 256 / per_row;
        const size_t lds = sizeof(float) * ((size_t)rb * per_row + (size_t)rb * (p.padded / p.group));
        if (lds > 64 * 1024) return hipErrorInvalidValue;
        rn_launch(cb_float_vector_kernel, dim3((p.rows + rb - 1) / rb, count), dim3(256), lds, stream, p, x, y, rb, nl);
    }
    return hipGetLastError();
}

hipError_t launch_codebook_product(const CodebookParams& p, const float* x, int count, float* y, int32_t* acc,
                                   hipStream_t stream) {
    if (count < 1 || p.rows < 1 || p.cpr < 1 || p.cpr > 1024) return hipErrorInvalidValue;
    switch (p.bits) {
        case 2: return launch_product_b<2, kPanel>(p, x, count, y, acc, stream);
        case 4: return launch_product_b<4, kPlane>(p, x, count, y, acc, stream);
        case 5: return launch_product_b<5, kPlane>(p, x, count, y, acc, stream);
        default: return hipErrorInvalidValue;
    }
}

namespace {

template <int BITS, int GROUP, int FORM>
hipError_t launch_jobs_t(CodebookJobs jobs, int n, hipStream_t stream) {
    const CodebookParams& p = jobs.job[0].p;
    const int nl = product_loads(p), R = product_rows(p);
    const size_t lds = product_lds(p, 1, R);
    if (lds > kProductMaxLds) return hipErrorInvalidValue;
    const int groups = (p.rows + 4 * R - 1) / (4 * R);
    const int iters = max(1, min(max(4, p.padded / 1024), groups / 512));
    for (int i = 0; i < n; ++i) {
        jobs.job[i].p.rows_per_block = R;
        jobs.job[i].p.iters = iters;
    }
    const dim3 grid((groups + iters - 1) / iters, 1, n);
    if (nl == 8)
        rn_launch(cb_product_jobs_kernel<BITS, GROUP, FORM, 8>, grid, dim3(256), lds, stream, jobs);
    else
        rn_launch(cb_product_jobs_kernel<BITS, GROUP, FORM, 16>, grid, dim3(256), lds, stream, jobs);
    return hipGetLastError();
}

template <int BITS, int FORM>
hipError_t launch_jobs_b(const CodebookJobs& jobs, int n, hipStream_t stream) {
    switch (jobs.job[0].p.group) {
        case 64: return launch_jobs_t<BITS, 64, FORM>(jobs, n, stream);
        case 128: return launch_jobs_t<BITS, 128, FORM>(jobs, n, stream);
        case 256: return launch_jobs_t<BITS, 256, FORM>(jobs, n, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_codebook_product_jobs(const CodebookJobs& jobs, int n, hipStream_t stream) {
    if (n < 1 || n > kCodebookJobs) return hipErrorInvalidValue;
    const CodebookParams& p = jobs.job[0].p;
    if (p.rows < 1 || p.cpr < 1 || p.cpr > 1024) return hipErrorInvalidValue;
    for (int i = 1; i < n; ++i) {
        const CodebookParams& q = jobs.job[i].p;
        if (q.bits != p.bits || q.group != p.group || q.padded != p.padded || q.rows != p.rows || q.cpr != p.cpr)
            return hipErrorInvalidValue;
    }
    switch (p.bits) {
        case 2: return launch_jobs_b<2, kPanel>(jobs, n, stream);
        case 4: return launch_jobs_b<4, kPlane>(jobs, n, stream);
        case 5: return launch_jobs_b<5, kPlane>(jobs, n, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_codebook_rotate(const float* x, int count, int columns, int padded, int group, float scale,
                                  float* rotated, hipStream_t stream) {
    if (count < 1 || padded % group != 0 || columns > padded) return hipErrorInvalidValue;
    const long long runs = (long long)count * (padded / 16);
    const dim3 grid((unsigned)((runs + 255) / 256));
    switch (group) {
        case 64: rn_launch(cb_rotate_kernel<64>, grid, dim3(256), 0, stream, x, count, columns, padded, scale, rotated); break;
        case 128: rn_launch(cb_rotate_kernel<128>, grid, dim3(256), 0, stream, x, count, columns, padded, scale, rotated); break;
        case 256: rn_launch(cb_rotate_kernel<256>, grid, dim3(256), 0, stream, x, count, columns, padded, scale, rotated); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_codebook_dequantise(const CodebookParams& p, int row, float* out, hipStream_t stream) {
    const int threads = ((p.padded / 16 + 63) / 64) * 64;
    if (row < 0 || row >= p.rows || threads > 1024) return hipErrorInvalidValue;
#define RN_DQ(B, GR) rn_launch(cb_dequantise_kernel<B, GR>, dim3(1), dim3(threads), 0, stream, p, row, out)
    switch (p.bits * 1000 + p.group) {
        case 1064: RN_DQ(1, 64); break;
        case 1128: RN_DQ(1, 128); break;
        case 1256: RN_DQ(1, 256); break;
        case 3064: RN_DQ(3, 64); break;
        case 3128: RN_DQ(3, 128); break;
        case 3256: RN_DQ(3, 256); break;
        case 2064: RN_DQ(2, 64); break;
        case 2128: RN_DQ(2, 128); break;
        case 2256: RN_DQ(2, 256); break;
        case 4064: RN_DQ(4, 64); break;
        case 4128: RN_DQ(4, 128); break;
        case 4256: RN_DQ(4, 256); break;
        case 5064: RN_DQ(5, 64); break;
        case 5128: RN_DQ(5, 128); break;
        case 5256: RN_DQ(5, 256); break;
        default: return hipErrorInvalidValue;
    }
#undef RN_DQ
    return hipGetLastError();
}

}  // namespace rn
