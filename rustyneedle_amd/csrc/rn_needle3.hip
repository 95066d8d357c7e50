// rn_needle3.hip — the Needle 3 token step (crates/model/src) on gfx950: the
// model read from a .cact archive in its canonical order (crates/cact/src/
// layout.rs:176-257), Session::push / feed / logits (session.rs:58-165) and the
// probe heads (heads.rs:84-150), every float in the reference's order.
//
// Device memory
//   model   : every codebook matrix as its archive blob (rn_matrix); the float
//             tensors (norm gains, conv taps, Hadamard diagonals, factors and
//             condition matrices, lane tensors, engram taps, final gains, the
//             dense probe and query rows of the heads) in one allocation each;
//             the two permutations as int32.
//   session : per layer the int8 cache, keys and values [kv][capacity][64]
//             with their scales [kv][capacity], and the conv-tap ring
//             [taps][q | k | v] (slot = position mod taps); per engram site
//             the ring of raw values [(taps - 1) * dilation + 1][d_model]; two
//             lane streams [lanes][d_model]; the cells [active + 1][d_model];
//             the head accumulators; the rotary table [capacity][32] (host
//             cosf / sinf, as the reference's sin_cos); scratch.
//
// Kernels of one push (host-driven, on the session's stream)
//   n3_stream_init    embedding row times sqrt(d) into every lane, cell 0;
//   n3_gather         engram: the tables' rows of the hashed slots, dequantised
//                     and fake-quantised (engram.rs:66-82);
//   n3_engram_conv    the value taps over the site's ring (engram.rs:84-111);
//   lanes route       rn_lanes (lanes.rs:48-84);
//   n3_block_in       add_engram (session.rs:175-188), the input norm, the fake
//                     quantisation and the rotation before the projections;
//   n3_qkv            conv taps (attention.rs:84-94), q/k norms, rotary, the
//                     per-head int8 codes and the cache append;
//   n3_attend         attend_head per query head (kernels/src/attention.rs:
//                     53-80 as the aarch64 build runs it) times sigmoid(gate);
//   n3_fake_quantise  the gated attention, fake-quantised and rotated for the
//                     output projection;
//   n3_block_out      post norm and gate, the Hadamard MLP (hadamard.rs:55-107,
//                     three 32 x 32 Kronecker products), block delta, lane
//                     combine and the cell (lanes.rs:86-104);
//   n3_final          lane mean and the final norm;
//   n3_observe        the heads' online softmax (heads.rs:138-155).
// The products are rn_codebook.hip's launches on rotated inputs; a layer's
// q, k, v and gate projections are one stacked matrix (one launch).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <new>
#include <string>
#include <type_traits>
#include <vector>

#include "../../include/rustyneedle.h"
#include "rn_device.hpp"
#include "rn_internal.hpp"
#include "rn_matrix.hpp"

namespace rn {

constexpr int kN3Block = 1024;
constexpr int kN3MaxWidth = 4096;     // stream, gathered rows, attention width
constexpr int kN3MaxAttend = 8192;    // positions one head attends
constexpr int kN3Head = 64;           // qk_head_dim = v_head_dim
constexpr int kN3MaxTables = 16;
constexpr int kN3Hadamard = 1024;     // 32 x 32

namespace {

// The maximum over the block (every thread calls; all get the result). With
// TAIL false the caller's next barrier must come before red is written again.
// LDS: the barriers wait for LDS operations only (callers whose threads share
// data through LDS only; global loads in flight stay in flight).
template <bool TAIL = true, bool LDS = false>
__device__ float n3_block_max(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = (blockDim.x + 63) >> 6;
    v = wave_max(v);
    if (lane == 0) red[wave] = v;
    if constexpr (LDS) lds_barrier(); else __syncthreads();
    // the waves' maxima (at most 16) on a row of lanes (the rest repeat the
    // last), joined inside the row
    float r = red[min(lane, waves - 1)];
    r = fmaxf(r, lane_xor<1>(r));
    r = fmaxf(r, lane_xor<2>(r));
    r = fmaxf(r, lane_xor<4>(r));
    r = fmaxf(r, lane_xor<8>(r));
    r = lane_float(r, 0);
    if (TAIL) {
        if constexpr (LDS) lds_barrier(); else __syncthreads();
    }
    return r;
}

// Sequential folds s = s + f(a[i], b[i]) over i = 0..count-1 at a stride, in
// order; the loads of sixteen elements are issued before their adds, so the
// chain waits on the adds and not on each load.
template <bool SQUARE>
__device__ __forceinline__ float n3_fold(float s, const float* a, const float* b, int count, int stride,
                                         int b_stride = -1) {
    const int sb = b_stride < 0 ? stride : b_stride;
    int i = 0;
    for (; i + 32 <= count; i += 32) {
        float x[32], y[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            x[j] = a[(size_t)(i + j) * stride];
            y[j] = SQUARE ? x[j] : b[(size_t)(i + j) * sb];
        }
#pragma unroll
        for (int j = 0; j < 32; ++j) s = s + x[j] * y[j];
    }
    for (; i < count; ++i) {
        const float x = a[(size_t)i * stride];
        s = s + x * (SQUARE ? x : b[(size_t)i * sb]);
    }
    return s;
}

// s + q[0].x + q[0].y + ... in order over `count` float4 values in LDS (a
// chain of dependent adds): three register sets of four values in turn, the
// loads of the set two ahead issued before the current set's adds, so that the
// chain waits on the adds and not on the LDS. The loads are issued
// unconditionally (the last set again past the end) and kept ahead of the adds
// by a scheduling barrier; at most twelve are in flight (the LDS counter
// holds fifteen), so the wait before a set's adds leaves the eight newer ones
// outstanding.
__device__ __forceinline__ float n3_chain4(const float4* q, int count, float s = 0.0f) {
    auto add4 = [&](const float4 (&v)[4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s = s + v[j].x;
            s = s + v[j].y;
            s = s + v[j].z;
            s = s + v[j].w;
        }
    };
    const int full = count / 4 * 4, last = full - 4;
    auto load4 = [&](float4 (&v)[4], int k) {
        k = min(k, last);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = q[k + j];
        __builtin_amdgcn_sched_barrier(0);  // issued here, ahead of the adds
    };
    if (full > 0) {
        // no scalar load in flight (those return out of order and would make
        // every wait below a full one)
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        float4 a[4], b[4], c[4];
        load4(a, 0);
        load4(b, 4);
        for (int k = 0;;) {
            load4(c, k + 8);
            add4(a);
            k += 4;
            if (k >= full) break;
            load4(a, k + 8);
            add4(b);
            k += 4;
            if (k >= full) break;
            load4(b, k + 8);
            add4(c);
            k += 4;
            if (k >= full) break;
        }
    }
    for (int k = full; k < count; ++k) {
        const float4 t = q[k];
        s = s + t.x;
        s = s + t.y;
        s = s + t.z;
        s = s + t.w;
    }
    return s;
}

// ops.rs:7-17 over n values in LDS: eight strided lanes, summed in lane order,
// then the tail. Every thread calls; all get the result. With `sq` (LDS
// scratch of n + 64 floats, 16-byte aligned, n / 8 a multiple of 4) the squares
// are first computed by every thread into sq, lane j's at row j (stride n / 8
// + 8, so the writes of a wave fall in distinct banks), and the eight chains
// only add, four squares a read.
__device__ float n3_sum_of_squares(const float* v, int n, float* red, float* sq = nullptr) {
    const int tid = threadIdx.x, n8 = n / 8;
    if (sq != nullptr && (n8 & 3) == 0) {
        const int stride = n8 + 8;
        for (int i = tid; i < n8 * 8; i += blockDim.x) {
            const float x = v[i];
            sq[(i & 7) * stride + (i >> 3)] = x * x;
        }
        lds_barrier();
        if (tid < 8) {
            red[tid] = n3_chain4(reinterpret_cast<const float4*>(sq + tid * stride), n8 / 4);
        }
    } else if (tid < 8) {
        red[tid] = n3_fold<true>(0.0f, v + tid, nullptr, n8, 8);
    }
    lds_barrier();
    float total = 0.0f;
    for (int j = 0; j < 8; ++j) total = total + red[j];
    float tail = -0.0f;
    for (int i = n8 * 8; i < n; ++i) tail = tail + v[i] * v[i];
    lds_barrier();
    return total + tail;
}

// ops.rs:44-58: out = ((1 + gain) * x) * inverse (out may be x)
__device__ void n3_norm(const float* x, const float* gain, int n, float* out, float* red, float* sq = nullptr) {
    const float mean_square = n3_sum_of_squares(x, n, red, sq) / (float)n;
    const float inverse = reciprocal(sqrtf(mean_square + 1e-6f));
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = ((1.0f + gain[i]) * x[i]) * inverse;
    __syncthreads();
}

// n3_norm for n <= blockDim.x with thread i's gain in a register
__device__ void n3_norm_gain(const float* x, float gain, int n, float* out, float* red, float* sq) {
    const float mean_square = n3_sum_of_squares(x, n, red, sq) / (float)n;
    const float inverse = reciprocal(sqrtf(mean_square + 1e-6f));
    const int i = threadIdx.x;
    if (i < n) out[i] = ((1.0f + gain) * x[i]) * inverse;
    lds_barrier();
}

// ops.rs:60-66
__device__ void n3_unit_rms(const float* x, int n, float* out, float* red, float* sq = nullptr) {
    const float inverse = reciprocal(sqrtf(n3_sum_of_squares(x, n, red, sq) / (float)n + 1e-6f));
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * inverse;
    __syncthreads();
}

// ops.rs:120-125 in place over LDS; the quotient v / scale without a division
// (quotients<1>: the same rounding), NaN kept as the reference keeps it
__device__ void n3_fake_quantise(float* v, int n, float* red) {
    float peak = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) peak = fmaxf(peak, fabsf(v[i]));
    peak = n3_block_max<false>(peak, red);  // red is next written after the barrier below
    const float scale = int8_scale_from_peak(peak);
    for (int base = 0; base < n; base += blockDim.x) {
        if (base + (int)(threadIdx.x & ~63u) >= n) break;  // a wave past the values
        const int i = base + threadIdx.x;
        const float x = v[min(i, n - 1)];
        float y;
        quotients<1>(&x, scale, &y);
        float q = __builtin_rintf(y);
        q = q < -128.0f ? -128.0f : (q > 127.0f ? 127.0f : q);
        if (i < n) v[i] = q * scale;
    }
    __syncthreads();
}

typedef __attribute__((address_space(3))) void n3_lds_void;
typedef __attribute__((address_space(1))) void n3_global_void;

// the level index of element e of a packed row (LSB first; 3-bit indices may
// straddle two bytes)
__device__ __forceinline__ int n3_index(const uint8_t* row, int e, int ib) {
    const int bit = e * ib;
    uint32_t raw = row[bit / 8];
    if ((bit % 8) + ib > 8) raw |= (uint32_t)row[bit / 8 + 1] << 8;
    return (raw >> (bit % 8)) & ((1 << ib) - 1);
}

// QuantisedMatrix::prepare (matrix.rs:123-128) in LDS: v [padded] (zero past
// the columns) rotated group by group (walsh.rs:41-76): butterflies of span 1,
// 2, 4, ... (low a + b, high a - b), then every value times `scale`.
__device__ void n3_rotate(float* v, int padded, int group, float scale) {
    const int half = group / 2;
    for (int span = 1; span < group; span *= 2) {
        for (int q = threadIdx.x; q < padded / 2; q += blockDim.x) {
            const int g = q / half, w = q - g * half;
            const int lo = g * group + (w / span) * 2 * span + (w % span), hi = lo + span;
            const float a = v[lo], b = v[hi];
            v[lo] = a + b;
            v[hi] = a - b;
        }
        __syncthreads();
    }
    for (int i = threadIdx.x; i < padded; i += blockDim.x) v[i] = v[i] * scale;
    __syncthreads();
}

// dst[i] = src[i] for i < n, eight loads a thread issued before their stores
// (the stores may alias the loads as far as the compiler knows)
__device__ void n3_copy(float* dst, const float* src, int n) {
    for (int base = 0; base < n; base += 8 * blockDim.x) {
        float t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = base + j * blockDim.x + threadIdx.x;
            t[j] = i < n ? src[i] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = base + j * blockDim.x + threadIdx.x;
            if (i < n) dst[i] = t[j];
        }
    }
}

}  // namespace

// ---- kernels ---------------------------------------------------------------

// tokens[position] = *source, or the host's token when source is null
constexpr int kN3FeedChunk = 256;  // tokens a batched feed runs together

// the ids of a run of tokens, passed by value
struct N3TokenRun {
    uint32_t ids[kN3FeedChunk];
};

__global__ void n3_set_tokens_kernel(uint32_t* tokens, int position, int count, N3TokenRun run) {
    for (int i = threadIdx.x; i < count; i += blockDim.x) tokens[position + i] = run.ids[i];
}

// session.rs:86-97: the embedding row of tokens[position] (dequantise_row,
// matrix.rs:140-153: level * norm, then each group's Walsh-Hadamard transform
// in registers, lane u holding run u) times sqrt(d) into every lane; cell 0 is
// their lane mean (session.rs:190-200). One block of 64 * ceil(runs / 64) a
// token: block b embeds position + b into stream + b * stream_stride and
// cell + b * cell_stride (prefill.rs:21-29 for a run of tokens). With `set`
// (one token) the token is *source (the greedy argmax) or `value`, and the
// block records it at tokens[position].
__device__ __forceinline__ void n3_embed_body(const CodebookParams& c, uint32_t token, int d, int lanes, float scale,
                                              float* stream, float* cell) {
    const int u = threadIdx.x, runs = c.padded / 16, rpg = c.group / 16, G = c.padded / c.group;
    const int ib = c.bits == 5 ? 2 : c.bits;
    const bool valid = u < runs;
    const uint8_t* row = c.packed + (size_t)token * c.row_bytes;
    const float norm = valid ? __half2float(__ushort_as_half(c.norms[(size_t)token * G + (16 * u) / c.group])) : 0.0f;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = valid ? c.levels[n3_index(row, 16 * u + i, ib)] * norm : 0.0f;
#pragma unroll
    for (int span = 1; span < 16; span *= 2)
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if ((i & span) == 0) {
                const float a = x[i], b = x[i + span];
                x[i] = a + b;
                x[i + span] = a - b;
            }
    // spans 16 .. group / 2 with the partner lane u ^ (span / 16) (every lane active)
    auto level = [&](auto m) {
        const bool high = (u & decltype(m)::value) != 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float q = lane_xor<decltype(m)::value>(x[i]);
            x[i] = high ? q - x[i] : x[i] + q;
        }
    };
    if (rpg > 1) level(std::integral_constant<int, 1>{});
    if (rpg > 2) level(std::integral_constant<int, 2>{});
    if (rpg > 4) level(std::integral_constant<int, 4>{});
    if (rpg > 8) level(std::integral_constant<int, 8>{});
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int e = 16 * u + i;
        if (!valid || e >= d) continue;
        const float v = (x[i] * c.wht_scale) * scale;
        float mean = 0.0f;
        for (int l = 0; l < lanes; ++l) {
            stream[(size_t)l * d + e] = v;
            mean = mean + v / (float)lanes;
        }
        cell[e] = mean;
    }
}

__global__ __launch_bounds__(1024) void n3_embed_kernel(CodebookParams c, uint32_t* tokens, int position, int d,
                                                        int lanes, float scale, float* stream, float* cell,
                                                        int stream_stride, int cell_stride, int set,
                                                        const uint32_t* source, uint32_t value) {
    const uint32_t token = set ? (source != nullptr ? *source : value) : tokens[position + blockIdx.x];
    if (set && threadIdx.x == 0) tokens[position] = token;
    n3_embed_body(c, token, d, lanes, scale, stream + (size_t)blockIdx.x * stream_stride,
                  cell + (size_t)blockIdx.x * cell_stride);
}

struct N3GatherParams {
    CodebookParams tables;
    int count, sub, slots, position;
    const uint32_t* tokens;  // the session's tokens [capacity]
    int heads_per_order, stride;
    int orders[4];
    float* out;  // [count * sub] a position, out_stride apart
    int out_stride;
    // with `rotated`: prepare for the key matrix (matrix.rs:123-128: zero to
    // rpadded, each group of rgroup rotated, times rwht) into rotated [rpadded]
    // instead of writing out
    float* rotated;
    int rpadded, rgroup;
    float rwht;
};

constexpr int kN3MaxSites = 4;  // engram sites one launch serves

struct N3GatherSites {
    N3GatherParams site[kN3MaxSites];
    int sites;  // blocks 0 .. sites - 1 (blockIdx.y) gather; with `embed`, block `sites` embeds
    // the push's token: *source (the greedy argmax) or value, recorded at
    // tokens[position] by the embedding block; the gathers take it from here
    int embed;
    CodebookParams table;
    uint32_t* tokens;
    int position, d, lanes;
    float scale;
    float *stream, *cell;
    const uint32_t* source;
    uint32_t value;
};

// engram.rs:66-82: row table * slots + index of each table (zeros while the
// position is shorter than the table's order), dequantised (matrix.rs:140-153),
// then fake_quantise_int8 over the whole gathered vector. Block b gathers
// position p.position + b (engram.rs:122-133 for a run of positions).
__global__ __launch_bounds__(kN3Block) void n3_gather_kernel(N3GatherSites sites) {
    __shared__ float buf[kN3MaxWidth];
    __shared__ float red[32];
    __shared__ int index_s[kN3MaxTables], order_s[kN3MaxTables];
    const bool mine = sites.embed != 0;  // the push's token comes from the launch
    const uint32_t now = mine ? (sites.source != nullptr ? *sites.source : sites.value) : 0u;
    if (mine && (int)blockIdx.y == sites.sites) {  // session.rs:86-97 for the push's token
        if (threadIdx.x == 0) sites.tokens[sites.position] = now;
        n3_embed_body(sites.table, now, sites.d, sites.lanes, sites.scale, sites.stream, sites.cell);
        return;
    }
    const N3GatherParams& p = sites.site[blockIdx.y];  // the site (one launch serves a push's sites)
    const CodebookParams& c = p.tables;
    const int n = p.count * p.sub, ib = c.bits == 5 ? 2 : c.bits, G = c.padded / c.group;
    const int position = p.position + (int)blockIdx.x;
    float* const out = p.out + (size_t)blockIdx.x * p.out_stride;
    if (threadIdx.x < p.count) {  // engram.rs:30-46: table (order o, head) hashes the last `order` tokens
        const int t = threadIdx.x, o = t / p.heads_per_order, head = t - o * p.heads_per_order;
        uint32_t acc = 0x9E3779B9u * (uint32_t)(o * p.stride + head + 1);
        for (int back = 0; back < p.orders[o]; ++back) {
            const uint32_t token = position >= back ? (mine && back == 0 ? now : p.tokens[position - back]) : 0u;
            acc = (acc ^ token) * 0x01000193u;
        }
        acc ^= acc >> 15;
        index_s[t] = (int)(acc % (uint32_t)p.slots);
        order_s[t] = p.orders[o];
    }
    __syncthreads();
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        const int t = e / p.sub, j = e - t * p.sub;
        float v = 0.0f;
        if (position + 1 >= order_s[t]) {
            const int row = t * p.slots + index_s[t];
            const float norm = __half2float(__ushort_as_half(c.norms[(size_t)row * G + j / c.group]));
            v = c.levels[n3_index(c.packed + (size_t)row * c.row_bytes, j, ib)] * norm;
        }
        buf[e] = v;
    }
    __syncthreads();
    n3_rotate(buf, n, c.group, c.wht_scale);  // each table row's groups (dequantise_row)
    n3_fake_quantise(buf, n, red);
    if (p.rotated != nullptr) {
        for (int e = n + threadIdx.x; e < p.rpadded; e += blockDim.x) buf[e] = 0.0f;
        __syncthreads();
        n3_rotate(buf, p.rpadded, p.rgroup, p.rwht);
        for (int e = threadIdx.x; e < p.rpadded; e += blockDim.x) p.rotated[e] = buf[e];
    } else {
        for (int e = threadIdx.x; e < n; e += blockDim.x) out[e] = buf[e];
    }
}

// engram.rs:84-111: value = sum over taps of gain * the raw value `tap *
// dilation` back. Token t = blockIdx.y is position + t, its raw value at raw +
// t * width; a raw value `back` positions earlier comes from the same run when
// back <= t (engram.rs:140-153), else from the ring (slot position mod keep).
// With write_ring (one token) the raw value joins the ring here; a run's
// values join it afterwards (n3_ring_store_kernel), once every block has read.
struct N3ConvSites {
    const float* raw[kN3MaxSites];
    float* ring[kN3MaxSites];
    const float* taps[kN3MaxSites];
    float* value[kN3MaxSites];
};

__global__ void n3_engram_conv_kernel(N3ConvSites sites, int position, int keep, int ntaps, int dilation, int width,
                                      int write_ring) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y, pos = position + t, e = blockIdx.z;
    const float* const raw = sites.raw[e];
    float* const ring = sites.ring[e];
    const float* const taps = sites.taps[e];
    float* const value = sites.value[e];
    if (i >= width) return;
    const float r = raw[(size_t)t * width + i];
    if (write_ring) ring[(size_t)(pos % keep) * width + i] = r;
    float v = 0.0f;
    for (int tap = 0; tap < ntaps; ++tap) {
        const int back = tap * dilation;
        if (pos < back) continue;
        const float sample = back == 0 ? r
                             : back <= t ? raw[(size_t)(t - back) * width + i]
                                         : ring[(size_t)((pos - back) % keep) * width + i];
        v = v + taps[(size_t)tap * width + i] * sample;
    }
    value[(size_t)t * width + i] = v;
}

// The last min(count, keep) rows of a run of positions [position, position +
// count) into their ring slots (slot position mod keep, ring_stride apart):
// the history the next position's taps read (engram.rs:155-159,
// attention.rs:265-273).
__global__ void n3_ring_store_kernel(const float* rows, int row_stride, int count, int position, int keep, int width,
                                     float* ring, int ring_stride) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x, t = count - min(count, keep) + (int)blockIdx.y;
    if (i >= width) return;
    ring[(size_t)((position + t) % keep) * ring_stride + i] = rows[(size_t)t * row_stride + i];
}

struct N3BlockInParams {
    const float* input;   // the routed input [d]
    const float* key;     // engram key [d] or null
    const float* value;   // engram value [d]
    const float* norm_in;
    int d;
    float* x;             // [d]
    int padded, group;    // of the projections
    float wht_scale;
    float* rotated;       // [padded] the fake-quantised norm of x, rotated (prepare)
};

// session.rs:112-118 with add_engram (session.rs:175-188).
__global__ __launch_bounds__(kN3Block) void n3_block_in_kernel(N3BlockInParams p) {
    __shared__ float xs[kN3MaxWidth], ta[kN3MaxWidth], tb[kN3MaxWidth];
    __shared__ float red[32];
    __shared__ float alpha_s;
    const int d = p.d;
    for (int i = threadIdx.x; i < d; i += blockDim.x) xs[i] = p.input[i];
    __syncthreads();
    if (p.key != nullptr) {
        n3_unit_rms(xs, d, ta, red);
        for (int i = threadIdx.x; i < d; i += blockDim.x) tb[i] = p.key[i];
        __syncthreads();
        n3_unit_rms(tb, d, tb, red);
        if (threadIdx.x == 0) {  // Iterator::sum: in order from -0.0
            const float dot = n3_fold<false>(-0.0f, ta, tb, d, 1);
            alpha_s = libm_sigmoid(dot / sqrtf((float)d));
        }
        __syncthreads();
        const float alpha = alpha_s;
        for (int i = threadIdx.x; i < d; i += blockDim.x) xs[i] = xs[i] + alpha * p.value[i];
        __syncthreads();
    }
    n3_norm(xs, p.norm_in, d, ta, red);
    n3_fake_quantise(ta, d, red);
    for (int i = d + threadIdx.x; i < p.padded; i += blockDim.x) ta[i] = 0.0f;
    __syncthreads();
    n3_rotate(ta, p.padded, p.group, p.wht_scale);
    for (int i = threadIdx.x; i < d; i += blockDim.x) p.x[i] = xs[i];
    for (int i = threadIdx.x; i < p.padded; i += blockDim.x) p.rotated[i] = ta[i];
}

struct N3QkvParams {
    const float* prod;     // q | k | v | gate projections of this token
    float* hist;           // conv-tap ring [taps][q | k | v]
    const float* taps[3];  // [taps][width] for q, k, v
    int ntaps, position, H, KV, cap;
    const float* q_norm;
    const float* k_norm;
    const float* cos_row;  // [32] at this position
    const float* sin_row;
    int8_t* qcodes;        // [H][64]
    float* qscales;        // [H]
    int8_t* keys;          // [KV][cap][64]
    float* key_scales;     // [KV][cap]
    int8_t* values;
    float* value_scales;
    int prod_stride;       // a run of tokens: token t's projections at prod + t * prod_stride
    int run;               // a run: taps of earlier tokens of the run from prod, the ring left alone
};

// attention.rs:110-141: conv taps over the raw q/k/v ring, per-head norms and
// rotary for q and k, int8 codes per head, the cache append. One wave per head
// (blocks 0..H-1 the queries, then the key and value heads) and token
// (blockIdx.y: position + t; attention.rs:242-318 for a run of tokens, whose
// raw rows join the ring afterwards, n3_ring_store_kernel).
__global__ __launch_bounds__(64) void n3_qkv_kernel(N3QkvParams p) {
    __shared__ float v_s[kN3Head];
    __shared__ float red[8];
    const int b = blockIdx.x, lane = threadIdx.x, t = blockIdx.y;
    const int which = b < p.H ? 0 : (b < p.H + p.KV ? 1 : 2);
    const int h = which == 0 ? b : (which == 1 ? b - p.H : b - p.H - p.KV);
    const int qw = p.H * kN3Head, kw = p.KV * kN3Head, total = qw + 2 * kw;
    const int width = which == 0 ? qw : kw, off = which == 0 ? 0 : (which == 1 ? qw : qw + kw);
    const int col = h * kN3Head + lane;
    const int position = p.position + t;
    const float* const prod = p.prod + (size_t)t * p.prod_stride;
    const float* const cos_row = p.cos_row + (size_t)t * 32;
    const float* const sin_row = p.sin_row + (size_t)t * 32;
    const float* const taps = which == 0 ? p.taps[0] : (which == 1 ? p.taps[1] : p.taps[2]);
    const float raw = prod[off + col];
    float v = raw;
    if (p.ntaps > 0) {
        if (!p.run) p.hist[(size_t)(position % p.ntaps) * total + off + col] = raw;
        const int n = min(p.ntaps, position + 1);
        v = 0.0f;
        for (int tap = 0; tap < n; ++tap) {
            const float sample = tap == 0 ? raw
                                 : (p.run && tap <= t) ? prod[off + col - (ptrdiff_t)tap * p.prod_stride]
                                                       : p.hist[(size_t)((position - tap) % p.ntaps) * total + off + col];
            v = v + taps[(size_t)tap * width + col] * sample;
        }
    }
    if (which < 2) {
        // ops.rs:52-58 over the head, then ops.rs:131-141
        v_s[lane] = v;
        __syncthreads();
        if (lane < 8) {
            float s = 0.0f;
            for (int c = 0; c < kN3Head / 8; ++c) s = s + v_s[8 * c + lane] * v_s[8 * c + lane];
            red[lane] = s;
        }
        __syncthreads();
        float ss = 0.0f;
        for (int j = 0; j < 8; ++j) ss = ss + red[j];
        const float inverse = reciprocal(sqrtf(ss / (float)kN3Head + 1e-6f));
        const float* gain = which == 0 ? p.q_norm : p.k_norm;
        v = ((1.0f + gain[lane]) * v) * inverse;
        __syncthreads();
        v_s[lane] = v;
        __syncthreads();
        const int half = kN3Head / 2;
        if (lane < half) {
            const float a = v_s[lane], bb = v_s[lane + half];
            v = a * cos_row[lane] - bb * sin_row[lane];
        } else {
            const int i = lane - half;
            const float a = v_s[i], bb = v_s[lane];
            v = bb * cos_row[i] + a * sin_row[i];
        }
    }
    // ops.rs:112-118
    const float peak = wave_max(fabsf(v));
    const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    const int8_t code = (int8_t)quantise_one(v, scale);
    if (which == 0) {
        p.qcodes[(size_t)t * qw + col] = code;
        if (lane == 0) p.qscales[(size_t)t * p.H + h] = scale;
    } else {
        const size_t row = (size_t)h * p.cap + position;
        (which == 1 ? p.keys : p.values)[row * kN3Head + lane] = code;
        if (lane == 0) (which == 1 ? p.key_scales : p.value_scales)[row] = scale;
    }
}

struct N3AttendParams {
    const int8_t* qcodes;
    const float* qscales;
    const int8_t* keys;    // [KV][cap][64]
    const float* key_scales;
    const int8_t* values;
    const float* value_scales;
    const float* gate;     // [H][64] gate projections
    int cap, position, window, group;  // window: positions a non-global layer sees (0: all)
    float inverse_root;
    float* out;            // [H][64]
    int gate_stride;       // a run of tokens: token t's gates at gate + t * gate_stride
};

// kernels/src/attention.rs:53-80 for query head blockIdx.x of the token at
// position + blockIdx.y over positions [first, position + 1) (first from the
// window, attention.rs:171-177), then times sigmoid(gate)
// (attention.rs:147-149; attention.rs:319-330 for a run of tokens).
// Scores are exact; coefficients ((float)score * key_scale) * query_scale; the
// exponent total is the aarch64 build's: four lane sums over the first
// count - count % 4 positions (position p in lane p % 4, in order), added as
// (l0 + l1) + (l2 + l3), then the remaining positions in order
// (neon.rs:278-311). The weights round(c / (peak / 2047)) (half away from
// zero) times the value codes sum exactly in int32 (neon.rs:347-438).
__global__ __launch_bounds__(256) void n3_attend_kernel(N3AttendParams p) {
    __shared__ float c_s[kN3MaxAttend];  // scores, then the exponents
    __shared__ int part[16][kN3Head];
    __shared__ float red[8];
    __shared__ float lanes_s[4];
    const int t = blockIdx.y, total_positions = p.position + t + 1;
    const int first = p.window > 0 && total_positions > p.window ? total_positions - p.window : 0;
    const int8_t* const qcodes = p.qcodes + (size_t)t * gridDim.x * kN3Head;
    const float* const gate = p.gate + (size_t)t * p.gate_stride;
    float* const out = p.out + (size_t)t * gridDim.x * kN3Head;
    const int h = blockIdx.x, tid = threadIdx.x, kvh = h / p.group, count = total_positions - first;
    const float query_scale = p.qscales[(size_t)t * gridDim.x + h] * p.inverse_root;
    int4 q[4];
    const int4* qs = reinterpret_cast<const int4*>(qcodes + (size_t)h * kN3Head);
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = qs[i];
    const int8_t* kbase = p.keys + ((size_t)kvh * p.cap + first) * kN3Head;
    const float* ks = p.key_scales + (size_t)kvh * p.cap + first;
    const float* vs = p.value_scales + (size_t)kvh * p.cap + first;
    float peak = -INFINITY;
    for (int pp = tid; pp < count; pp += 256) {
        const int4* k = reinterpret_cast<const int4*>(kbase + (size_t)pp * kN3Head);
        int score = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) score = dot16(q[i], k[i], score);
        const float c = ((float)score * ks[pp]) * query_scale;
        c_s[pp] = c;
        peak = fmaxf(peak, c);
    }
    peak = n3_block_max(peak, red);
    // the exponents, and the peak of the coefficients e * value_scale
    float cpeak = 0.0f;
    for (int pp = tid; pp < count; pp += 256) {
        const float e = fast_exp(c_s[pp] - peak);
        c_s[pp] = e;
        cpeak = fmaxf(cpeak, fabsf(e * vs[pp]));
    }
    cpeak = n3_block_max(cpeak, red);  // its barrier orders the exponents before the reads below
    const int vector_count = count - count % 4;
    if (tid < 4) {
        float s = 0.0f;
        int pp = tid;
        for (; pp + 64 <= vector_count; pp += 64) {
            float e[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) e[j] = c_s[pp + 4 * j];
#pragma unroll
            for (int j = 0; j < 16; ++j) s = s + e[j];
        }
        for (; pp < vector_count; pp += 4) s = s + c_s[pp];
        lanes_s[tid] = s;
    }
    const float scale = cpeak / 2047.0f;
    const int dg = tid & 15, pc = tid >> 4;
    int acc[4] = {0, 0, 0, 0};
    if (cpeak > 0.0f) {
        const int8_t* vbase = p.values + ((size_t)kvh * p.cap + first) * kN3Head + 4 * dg;
        for (int pp = pc; pp < count; pp += 16) {
            const int w = (int)__builtin_roundf((c_s[pp] * vs[pp]) / scale);
            if (w == 0) continue;
            const int packed = *reinterpret_cast<const int*>(vbase + (size_t)pp * kN3Head);
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[k] += w * (int)(int8_t)(packed >> (8 * k));
        }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) part[pc][4 * dg + k] = acc[k];
    __syncthreads();
    if (tid < kN3Head) {
        int sum = 0;
        for (int c = 0; c < 16; ++c) sum += part[c][tid];
        float total = (lanes_s[0] + lanes_s[1]) + (lanes_s[2] + lanes_s[3]);
        for (int pp = vector_count; pp < count; ++pp) total = total + c_s[pp];
        float o = cpeak > 0.0f ? (float)sum * scale : 0.0f;
        o = o * reciprocal(total);
        o = o * libm_sigmoid(gate[(size_t)h * kN3Head + tid]);
        out[(size_t)h * kN3Head + tid] = o;
    }
}

// ops.rs:120-125 over n <= 4096 values (one block a vector: block b reads in +
// b * n), then, for group > 0, prepare for a matrix of that group and padded
// width (matrix.rs:123-128) into out + b * padded (else out + b * n)
__global__ __launch_bounds__(kN3Block) void n3_fake_quantise_kernel(const float* in, int n, int padded, int group,
                                                                    float wht_scale, float* out) {
    __shared__ float buf[kN3MaxWidth];
    __shared__ float red[32];
    in += (size_t)blockIdx.x * n;
    out += (size_t)blockIdx.x * (group > 0 ? padded : n);
    for (int i = threadIdx.x; i < n; i += blockDim.x) buf[i] = in[i];
    __syncthreads();
    n3_fake_quantise(buf, n, red);
    if (group > 0) {
        for (int i = n + threadIdx.x; i < padded; i += blockDim.x) buf[i] = 0.0f;
        __syncthreads();
        n3_rotate(buf, padded, group, wht_scale);
    } else {
        padded = n;
    }
    for (int i = threadIdx.x; i < padded; i += blockDim.x) out[i] = buf[i];
}

struct N3BlockOutParams {
    const float* attention;    // out projection [d]
    const float* post_norm;
    float gate;                // sigmoid(attention_gate)
    const float* pre_norm;
    const float *d1, *d2, *b2, *d3, *d4;
    const float* factors[6];   // w1a w1b w2a w2b w3a w3b, [32][32]
    const float* cond_v;       // [d][rank]
    const float* cond_u;       // [rank][1024]
    int rank;
    const int32_t* perm1;
    const int32_t* perm2;
    const float* x;            // block input after the attention input norm
    const float* input;        // routed input
    const float* post;         // [lanes]
    const float* residual;     // [lanes][lanes]
    const float* stream;       // [lanes][d]
    int d, lanes;
    float* next;               // [lanes][d]
    float* cell;               // [d]
};

// kronecker_apply for 32 x 32 factors (ops.rs:220-297): mixed = X . R, then
// out = L^T . mixed, each a chain of fused multiply-adds in index order.
// Every thread of the block calls (256 or more); x and out in LDS (distinct),
// mixed LDS scratch; x and left 16-byte aligned.
__device__ __forceinline__ void n3_kronecker32(const float* x, const float* left, const float* right, float* mixed, float* out) {
    // threads 0..255: column c of rows 4 q .. 4 q + 3, so that a column of the
    // right factor (stage one) or of the mixed matrix (stage two) read once
    // serves four outputs; each output's chain stays in index order
    const int tid = threadIdx.x, c = tid & 31, i0 = (tid >> 5) * 4;
    if (tid < 256) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 32; j += 4) {
            float r[4];
            float4 q[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) r[k] = right[(j + k) * 32 + c];
#pragma unroll
            for (int m = 0; m < 4; ++m) q[m] = *reinterpret_cast<const float4*>(x + (i0 + m) * 32 + j);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                acc[m] = __builtin_fmaf(r[0], q[m].x, acc[m]);
                acc[m] = __builtin_fmaf(r[1], q[m].y, acc[m]);
                acc[m] = __builtin_fmaf(r[2], q[m].z, acc[m]);
                acc[m] = __builtin_fmaf(r[3], q[m].w, acc[m]);
            }
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) mixed[(i0 + m) * 32 + c] = acc[m];
    }
    __syncthreads();
    if (tid < 256) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < 32; r += 4) {
            float mv[4];
            float4 l[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                mv[k] = mixed[(r + k) * 32 + c];
                l[k] = *reinterpret_cast<const float4*>(left + (r + k) * 32 + i0);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                acc[0] = __builtin_fmaf(mv[k], l[k].x, acc[0]);
                acc[1] = __builtin_fmaf(mv[k], l[k].y, acc[1]);
                acc[2] = __builtin_fmaf(mv[k], l[k].z, acc[2]);
                acc[3] = __builtin_fmaf(mv[k], l[k].w, acc[3]);
            }
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) out[(i0 + m) * 32 + c] = acc[m];
    }
    __syncthreads();
}

// LDS of the block tail: six Hadamard-sized arrays, the rank-8 condition rows
struct N3TailLds {
    float *xs, *a, *sc, *st, *mx, *modulation, *cv, *chains, *weights, *red;
    // a staged tail's inputs, copied into LDS: attention, x and input [3][d];
    // the six factors [6][1024]; the stream [lanes][d]; post [kMaxLanes] and
    // residual [kMaxLanes^2]
    float* tin;
    const float *factors, *stream, *lane;
};

// A thread's elementwise Hadamard tensors, read at kernel start so that their
// latency overlaps the work before the MLP.
struct N3TailPre {
    float d1, d2, b2, d3, d4, cond_u[8];
    float post_gain, pre_gain;  // element threadIdx.x of post_norm and pre_norm (0 past d)
    int perm1, perm2;
};

__device__ N3TailPre n3_tail_prefetch(const N3BlockOutParams& p) {
    const int tid = threadIdx.x;
    N3TailPre t;
    t.d1 = p.d1[tid];
    t.d2 = p.d2[tid];
    t.b2 = p.b2[tid];
    t.d3 = p.d3[tid];
    t.d4 = p.d4[tid];
    t.perm1 = p.perm1[tid];
    t.perm2 = p.perm2[tid];
    t.post_gain = p.post_norm[min(tid, p.d - 1)];
    t.pre_gain = p.pre_norm[min(tid, p.d - 1)];
#pragma unroll
    for (int r = 0; r < 8; ++r) t.cond_u[r] = r < p.rank ? p.cond_u[(size_t)r * kN3Hadamard + tid] : 0.0f;
    return t;
}

// session.rs:119-146 from the output projection: post norm, gated residual,
// the pre-Hadamard norm, HadamardWeights::apply, the block delta, the lane
// combine and the next cell; the next stream also into `keep` (LDS) when set.
// 1024 threads (the Hadamard size).
// STAGED: the inputs are LDS copies (l.tin, l.factors, l.stream, l.lane; cond_v
// of rank 8 in l.cv), read as LDS (the pointers' address space is fixed per
// instantiation), and the factors and cond_v may still be in flight (loads
// into LDS) until the condition products.
template <bool STAGED>
__device__ void n3_tail(const N3BlockOutParams& p, const N3TailLds& l, float* keep, const N3TailPre& pre) {
    float *xs = l.xs, *a = l.a, *sc = l.sc, *st = l.st, *mx = l.mx, *modulation = l.modulation;
    float *cv = l.cv, *weights = l.weights, *red = l.red;
    float(*chains)[8] = reinterpret_cast<float(*)[8]>(l.chains);
    const int tid = threadIdx.x, d = p.d;
    const float* const input = STAGED ? l.tin + 2 * d : p.input;
    const float* const stream = STAGED ? l.stream : p.stream;
    const float* const post = STAGED ? l.lane : p.post;
    const float* const residual = STAGED ? l.lane + kMaxLanes : p.residual;
    const float* factor[6];
#pragma unroll
    for (int f = 0; f < 6; ++f) factor[f] = STAGED ? l.factors + f * kN3Hadamard : p.factors[f];
    if (STAGED) {  // attention, x and (rank 8) cond_v already in LDS: work on them in place
        a = l.tin;
        xs = l.tin + d;
    } else {
        n3_copy(a, p.attention, d);
        n3_copy(xs, p.x, d);
        if (p.rank == 8) n3_copy(cv, p.cond_v, d * 8);
        __syncthreads();
    }
    n3_norm_gain(a, pre.post_gain, d, a, red, st);
    if (tid < d) xs[tid] = xs[tid] + p.gate * a[tid];
    lds_barrier();
    n3_norm_gain(xs, pre.pre_gain, d, a, red, st);  // a = pre
    if (STAGED) {  // the factors and cond_v, copied into LDS as the tail began
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    // condition weights (hadamard.rs:57-79): the products value * factor by
    // every thread, stored so that each of the 32 chains (lane j of rank r:
    // rows 4k + j in order) reads its products as consecutive float4 values
    // (chain c = 8 j + r at c * stride floats, stride the longest chain
    // rounded up to four, plus four where the 8192 floats of cv allow, so
    // that the 32 chains start in different banks); the chains then only add
    // (n3_chain4, the last values of a chain of n % 4 != 0 one at a time)
    if (p.rank == 8) {
        const int n4 = ((d + 3) / 4 + 3) / 4 * 4, stride = min(n4 + 4, kN3Hadamard / 4);
        float pv[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int e = tid + k * kN3Block;
            pv[k] = e < d * 8 ? a[e >> 3] * cv[e] : 0.0f;
        }
        lds_barrier();
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int e = tid + k * kN3Block;
            if (e < d * 8) {
                const int i = e >> 3, r = e & 7;
                cv[((i & 3) * 8 + r) * stride + (i >> 2)] = pv[k];
            }
        }
        lds_barrier();
        if (tid < 32) {
            const int j = tid >> 3, n = (d - j + 3) / 4;
            const float* q = cv + tid * stride;
            float sum = n3_chain4(reinterpret_cast<const float4*>(q), n / 4);
            for (int k = n / 4 * 4; k < n; ++k) sum = sum + q[k];
            chains[j][tid & 7] = sum;
        }
        lds_barrier();
        if (tid < 8) weights[tid] = (((0.0f + chains[0][tid]) + chains[1][tid]) + chains[2][tid]) + chains[3][tid];
    } else if (tid < p.rank) {
        float s = 0.0f;
        for (int i = 0; i < d; ++i) s = s + a[i] * p.cond_v[(size_t)i * p.rank + tid];
        weights[tid] = s;
    }
    __syncthreads();
    if (tid < 64) {  // ops.rs:92-101: the peak (order-free) and the exponentials by lane, the total in order
        const int R = p.rank;
        const float w = tid < R ? weights[tid] : -INFINITY;
        const float peak = wave_max(w);
        const float e = fast_exp(w - peak);
        float total = 0.0f;
        for (int r = 0; r < R; ++r) total = total + lane_float(e, r);
        const float inverse = reciprocal(total);
        if (tid < R) weights[tid] = e * inverse;
    }
    __syncthreads();
    {
        float m = 1.0f;
        if (p.rank <= 8) {
#pragma unroll
            for (int r = 0; r < 8; ++r)
                if (r < p.rank) m = m + weights[r] * pre.cond_u[r];
        } else {
            for (int r = 0; r < p.rank; ++r) m = m + weights[r] * p.cond_u[(size_t)r * kN3Hadamard + tid];
        }
        modulation[tid] = m;
        sc[tid] = (tid < d ? a[tid] : 0.0f) * pre.d1;
    }
    __syncthreads();
    n3_kronecker32(sc, factor[0], factor[1], mx, st);
    sc[tid] = silu(((pre.d2 * modulation[tid]) * st[pre.perm1]) + pre.b2);
    __syncthreads();
    n3_kronecker32(sc, factor[2], factor[3], mx, st);
    sc[tid] = st[pre.perm2] * pre.d3;
    __syncthreads();
    n3_kronecker32(sc, factor[4], factor[5], mx, st);
    mx[tid] = st[tid] * pre.d4;  // mlp
    __syncthreads();
    // block output, delta (lanes.rs:100-104), combine (lanes.rs:86-98), cell
    for (int i = tid; i < d; i += blockDim.x) {
        const float xo = xs[i] + mx[i];
        const float delta = xo - input[i];
        float mean = 0.0f;
        for (int ln = 0; ln < p.lanes; ++ln) {
            float o = 0.0f;
            for (int s = 0; s < p.lanes; ++s) o = o + residual[ln * p.lanes + s] * stream[(size_t)s * d + i];
            o = o + post[ln] * delta;
            p.next[(size_t)ln * d + i] = o;
            if (keep) keep[(size_t)ln * d + i] = o;
            mean = mean + o / (float)p.lanes;
        }
        p.cell[i] = mean;
    }
    __syncthreads();
}

__global__ __launch_bounds__(kN3Block) void n3_block_out_kernel(N3BlockOutParams p) {
    __shared__ __align__(16) float xs[kN3Hadamard], a[kN3Hadamard], sc[kN3Hadamard], st[kN3Hadamard], mx[kN3Hadamard];
    __shared__ float modulation[kN3Hadamard];
    __shared__ float chains[32];
    __shared__ float weights[64];
    __shared__ float red[32];
    __shared__ __align__(16) float cv[kN3Hadamard * 8];  // cond_v of rank 8
    const N3TailLds l{xs, a, sc, st, mx, modulation, cv, chains, weights, red, nullptr, nullptr, nullptr, nullptr};
    const N3TailPre pre = n3_tail_prefetch(p);
    n3_tail<false>(p, l, nullptr, pre);
}

// session.rs:141-144: lane mean and the final norm
__global__ __launch_bounds__(kN3Block) void n3_final_kernel(const float* stream, int d, int lanes, const float* gain,
                                                            float* hidden) {
    __shared__ float m[kN3MaxWidth];
    __shared__ float red[32];
    for (int i = threadIdx.x; i < d; i += blockDim.x) {
        float v = 0.0f;
        for (int l = 0; l < lanes; ++l) v = v + stream[(size_t)l * d + i] / (float)lanes;
        m[i] = v;
    }
    __syncthreads();
    n3_norm(m, gain, d, m, red);
    for (int i = threadIdx.x; i < d; i += blockDim.x) hidden[i] = m[i];
}

// ops.rs:19-30 by one block: eight strided lanes (threads 0..7), summed in lane
// order from -0.0, plus the tail from -0.0. All threads get the value.
__device__ float n3_dot_product(const float* a, const float* b, int n, float* red) {
    const int tid = threadIdx.x;
    if (tid < 8) red[tid] = n3_fold<false>(0.0f, a + tid, b + tid, n / 8, 8);
    __syncthreads();
    float total = -0.0f;
    for (int j = 0; j < 8; ++j) total = total + red[j];
    float tail = -0.0f;
    for (int i = n / 8 * 8; i < n; ++i) tail = tail + a[i] * b[i];
    __syncthreads();
    return total + tail;
}

constexpr int kN3MaxHeads = 4;  // probe heads one launch serves

struct N3ObserveHeads {
    const float* probes[kN3MaxHeads];
    float* peak[kN3MaxHeads];
    float* total[kN3MaxHeads];
    float* weighted[kN3MaxHeads];
    int k[kN3MaxHeads], width[kN3MaxHeads], first[kN3MaxHeads + 1];  // first slot (block) of each head
    int count;
};

// heads.rs:138-155: one block per slot (layer * k + probe) of each head
__global__ __launch_bounds__(256) void n3_observe_kernel(const float* cells, N3ObserveHeads hs) {
    __shared__ float red[8];
    __shared__ float rw[2];
    int hh = 0;
    for (int j = 1; j < hs.count; ++j) hh = (int)blockIdx.x >= hs.first[j] ? j : hh;
    const int h = __builtin_amdgcn_readfirstlane(hh);
    const int k = hs.k[h], width = hs.width[h];
    const float* const probes = hs.probes[h];
    float* const peak = hs.peak[h];
    float* const total = hs.total[h];
    float* const weighted = hs.weighted[h];
    const int slot = (int)blockIdx.x - hs.first[h], layer = slot / k;
    const float* cell = cells + (size_t)layer * width;
    const float dot = n3_dot_product(cell, probes + (size_t)slot * width, width, red);
    if (threadIdx.x == 0) {
        const float score = dot / sqrtf((float)width);
        const float old = peak[slot];
        const float pk = fmaxf(old, score);
        const float rescale = old == -INFINITY ? 0.0f : libm_expf(old - pk);
        const float weight = libm_expf(score - pk);
        total[slot] = total[slot] * rescale + weight;
        peak[slot] = pk;
        rw[0] = rescale;
        rw[1] = weight;
    }
    __syncthreads();
    const float rescale = rw[0], weight = rw[1];
    float* target = weighted + (size_t)slot * width;
    for (int i = threadIdx.x; i < width; i += blockDim.x) target[i] = target[i] * rescale + weight * cell[i];
}

// n3_observe_kernel over a run of tokens in order (prefill.rs:92-96): one
// block per slot; the run's scores first (ops.rs:19-30, 32 tokens at a time,
// eight lanes each), since they do not depend on the accumulator, then the
// online updates token by token (heads.rs:138-155).
__global__ __launch_bounds__(256) void n3_observe_run_kernel(const float* cells, int cell_stride, int count,
                                                             const float* probes, int k, int width, float* peak,
                                                             float* total, float* weighted) {
    __shared__ float score_s[kN3FeedChunk], rescale_s[kN3FeedChunk], weight_s[kN3FeedChunk];
    __shared__ float red[256];
    const int slot = blockIdx.x, layer = slot / k, tid = threadIdx.x;
    const float* probe = probes + (size_t)slot * width;
    const float* first_cell = cells + (size_t)layer * width;
    for (int t0 = 0; t0 < count; t0 += 32) {
        const int tt = t0 + (tid >> 3), j = tid & 7;
        if (tt < count) red[tid] = n3_fold<false>(0.0f, first_cell + (size_t)tt * cell_stride + j, probe + j, width / 8, 8);
        __syncthreads();
        if (tid < 32 && t0 + tid < count) {
            const float* cell = first_cell + (size_t)(t0 + tid) * cell_stride;
            float sum = -0.0f;
            for (int q = 0; q < 8; ++q) sum = sum + red[8 * tid + q];
            float tail = -0.0f;
            for (int i = width / 8 * 8; i < width; ++i) tail = tail + cell[i] * probe[i];
            score_s[t0 + tid] = (sum + tail) / sqrtf((float)width);
        }
        __syncthreads();
    }
    if (tid == 0) {
        float pk = peak[slot], tot = total[slot];
        for (int t = 0; t < count; ++t) {
            const float score = score_s[t], next = fmaxf(pk, score);
            const float rescale = pk == -INFINITY ? 0.0f : libm_expf(pk - next);
            const float weight = libm_expf(score - next);
            tot = tot * rescale + weight;
            pk = next;
            rescale_s[t] = rescale;
            weight_s[t] = weight;
        }
        peak[slot] = pk;
        total[slot] = tot;
    }
    __syncthreads();
    float* target = weighted + (size_t)slot * width;
    for (int i = tid; i < width; i += blockDim.x) {
        float w = target[i];
        for (int t = 0; t < count; ++t) w = w * rescale_s[t] + weight_s[t] * first_cell[(size_t)t * cell_stride + i];
        target[i] = w;
    }
}

// heads.rs:102-110: per slot, the average over the online total, unit_rms,
// times the slot's gain
__global__ __launch_bounds__(256) void n3_readout_kernel(const float* weighted, const float* total, const float* gain,
                                                         int width, float* readouts) {
    __shared__ float v[kN3MaxWidth];
    __shared__ float red[32];
    const int slot = blockIdx.x;
    const float inverse = reciprocal(total[slot]);
    for (int i = threadIdx.x; i < width; i += blockDim.x) v[i] = weighted[(size_t)slot * width + i] * inverse;
    __syncthreads();
    n3_unit_rms(v, width, v, red);
    const float g = gain[slot];
    for (int i = threadIdx.x; i < width; i += blockDim.x) readouts[(size_t)slot * width + i] = v[i] * g;
}

// heads.rs:111-124 for query blockIdx.x
__global__ __launch_bounds__(256) void n3_pool_kernel(const float* readouts, int slots, const float* query,
                                                      const float* row_bias, int width, float* pooled) {
    __shared__ float w[1024];
    __shared__ float red[8];
    const int q = blockIdx.x;
    const float root = sqrtf((float)width);
    for (int s = 0; s < slots; ++s) {
        const float dot = n3_dot_product(readouts + (size_t)s * width, query + (size_t)q * width, width, red);
        if (threadIdx.x == 0) w[s] = dot / root + row_bias[(size_t)q * slots + s];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float peak = -INFINITY;
        for (int s = 0; s < slots; ++s) peak = fmaxf(peak, w[s]);
        float t = 0.0f;
        for (int s = 0; s < slots; ++s) {
            w[s] = fast_exp(w[s] - peak);
            t = t + w[s];
        }
        const float inverse = reciprocal(t);
        for (int s = 0; s < slots; ++s) w[s] = w[s] * inverse;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < width; i += blockDim.x) {
        float o = 0.0f;
        for (int s = 0; s < slots; ++s) o = o + w[s] * readouts[(size_t)s * width + i];
        pooled[(size_t)q * width + i] = o;
    }
}

__global__ void n3_add_kernel(float* y, const float* bias, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = y[i] + bias[i];
}

// ---- the fused step: three kernels a layer -------------------------------------
//
//   n3_attention_kernel  one block a query head: the head's q, its kv head's k
//                        and v, and its gate rows of the stacked projection
//                        (integer path on the block's own group codes of the
//                        rotated input), conv taps, norms, rotary, codes, the
//                        cache append (the blocks of a kv group write the same
//                        bytes), attention and the gate;
//   n3_out_kernel        each block fake-quantises and rotates the gated
//                        attention itself, then 64 rows of the output
//                        projection;
//   n3_boundary_kernel   one block: the tail of a layer (n3_tail), the final
//                        norm after the last, or the routing of the next layer
//                        (its routing rows on the block's own group codes),
//                        add_engram, the input norm, fake quantisation and
//                        rotation.

// The int8 levels of four indices (one per byte of sel) from the sixteen-entry
// table in lut (v_perm_b32).
template <int IB>
__device__ __forceinline__ int n3_decode4(uint32_t sel, const uint32_t (&lut)[4]) {
    if constexpr (IB == 2) {
        return (int)__builtin_amdgcn_perm(0u, lut[0], sel);
    } else {
        const uint32_t s7 = sel & 0x07070707u;
        const uint32_t lo = __builtin_amdgcn_perm(lut[1], lut[0], s7);
        const uint32_t hi = __builtin_amdgcn_perm(lut[3], lut[2], s7);
        const uint32_t m = ((sel >> 3) & 0x01010101u) * 0xffu;
        return (int)((hi & m) | (lo & ~m));
    }
}

__device__ __forceinline__ int n3_b4(int a, int b, int c, int d) {
    return (a & 0xff) | ((b & 0xff) << 8) | ((c & 0xff) << 16) | ((d & 0xff) << 24);
}

// Pack sixteen codes of a run in the order its packed indices decode: for
// 2-bit dword k holds elements k, 4+k, 8+k, 12+k; for 4-bit dword 2h+k holds
// 8h+k, 8h+2+k, 8h+4+k, 8h+6+k.
__device__ __forceinline__ int4 n3_pack_codes(const int (&c)[16], int ib) {
    return ib == 2 ? make_int4(n3_b4(c[0], c[4], c[8], c[12]), n3_b4(c[1], c[5], c[9], c[13]),
                               n3_b4(c[2], c[6], c[10], c[14]), n3_b4(c[3], c[7], c[11], c[15]))
                   : make_int4(n3_b4(c[0], c[2], c[4], c[6]), n3_b4(c[1], c[3], c[5], c[7]),
                               n3_b4(c[8], c[10], c[12], c[14]), n3_b4(c[9], c[11], c[13], c[15]));
}

// One butterfly level across lanes: partner lane L ^ M holds the other half
// of each pair (low a + b, high a - b, walsh.rs:41-76).
template <int M>
__device__ __forceinline__ void n3_butterfly_lanes(float (&x)[4], bool high) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float q = lane_xor<M>(x[e]);
        x[e] = high ? q - x[e] : x[e] + q;
    }
}

// prepare and the per-group codes in one pass (matrix.rs:123-128 then
// panel.rs:52-66) over P values (zero past the columns) that load(L, x) gives
// four a lane, four lanes per run of 16 (groups of at most 256): lane L holds
// elements 4L .. 4L + 3;
// the Walsh-Hadamard butterflies (walsh.rs:41-76) of spans 1 and 2 in the lane, spans
// 4 .. group / 2 with the partner lane L ^ (span / 4) (low a + b, high a - b),
// scales, the group's peak over its group / 4 lanes, quotients without a
// division (quotients<4>: the codes of quantise_one), then the run's four
// lanes (a quad) exchange their codes by DPP broadcasts so that lane d of the
// run writes dword d of its plane-order int4. The exchanges between lanes are
// DPP moves and lane swaps (lane_xor), with every lane of the block active.
template <typename Load>
__device__ __forceinline__ void n3_codes_from(Load load, int P, int group, float wht_scale, int ib, int4* xq, float* xs) {
    const int lanes = P / 4, lpg = group / 4;
    int* xqw = reinterpret_cast<int*>(xq);
    for (int base = 0; base < lanes; base += blockDim.x) {
        if (base + (int)(threadIdx.x & ~63u) >= lanes) break;  // a wave past the runs
        const int L = base + threadIdx.x;
        const bool valid = L < lanes;
        float x[4];
        load(valid ? L : 0, x);
        float a0 = x[0], b0 = x[1], a1 = x[2], b1 = x[3];
        x[0] = a0 + b0;
        x[1] = a0 - b0;
        x[2] = a1 + b1;
        x[3] = a1 - b1;
        a0 = x[0], b0 = x[2], a1 = x[1], b1 = x[3];
        x[0] = a0 + b0;
        x[2] = a0 - b0;
        x[1] = a1 + b1;
        x[3] = a1 - b1;
        if (lpg > 1) n3_butterfly_lanes<1>(x, (L & 1) != 0);
        if (lpg > 2) n3_butterfly_lanes<2>(x, (L & 2) != 0);
        if (lpg > 4) n3_butterfly_lanes<4>(x, (L & 4) != 0);
        if (lpg > 8) n3_butterfly_lanes<8>(x, (L & 8) != 0);
        if (lpg > 16) n3_butterfly_lanes<16>(x, (L & 16) != 0);
        if (lpg > 32) n3_butterfly_lanes<32>(x, (L & 32) != 0);
        float peak = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[e] = x[e] * wht_scale;
            peak = fmaxf(peak, fabsf(x[e]));
        }
        if (lpg > 1) peak = fmaxf(peak, lane_xor<1>(peak));
        if (lpg > 2) peak = fmaxf(peak, lane_xor<2>(peak));
        if (lpg > 4) peak = fmaxf(peak, lane_xor<4>(peak));
        if (lpg > 8) peak = fmaxf(peak, lane_xor<8>(peak));
        if (lpg > 16) peak = fmaxf(peak, lane_xor<16>(peak));
        if (lpg > 32) peak = fmaxf(peak, lane_xor<32>(peak));
        const float scale = int8_scale_from_peak(peak);
        float y[4];
        quotients<4>(x, scale, y);
        const int w = n3_b4(code_of_quotient(y[0]), code_of_quotient(y[1]), code_of_quotient(y[2]),
                            code_of_quotient(y[3]));
        const int w0 = dpp_move<0x00>(w), w1 = dpp_move<0x55>(w), w2 = dpp_move<0xaa>(w), w3 = dpp_move<0xff>(w);
        const int d = L & 3;
        int out = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = ib == 2 ? 4 * j + d : 8 * (d >> 1) + 2 * j + (d & 1);
            const int src = e >> 2, ws = src == 0 ? w0 : src == 1 ? w1 : src == 2 ? w2 : w3;
            out |= ((ws >> (8 * (e & 3))) & 0xff) << (8 * j);
        }
        if (valid) {
            xqw[L] = out;
            if ((L & (lpg - 1)) == 0) xs[L / lpg] = scale;
        }
    }
}

// n3_codes_from over v [P] in LDS (16-byte aligned, zero past the columns)
__device__ __forceinline__ void n3_prepare_codes(const float* v, int P, int group, float wht_scale, int ib, int4* xq, float* xs) {
    n3_codes_from(
        [&](int L, float (&x)[4]) {
            const float4 t = reinterpret_cast<const float4*>(v)[L];
            x[0] = t.x;
            x[1] = t.y;
            x[2] = t.z;
            x[3] = t.w;
        },
        P, group, wht_scale, ib, xq, xs);
}

// ops.rs:120-125 for four values of a vector whose scale is known:
// round(value / scale) clamped to the int8 range, times scale (NaN kept)
__device__ __forceinline__ void n3_fake_quantise4(float (&x)[4], float scale) {
    float y[4];
    quotients<4>(x, scale, y);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float q = __builtin_rintf(y[e]);
        q = q < -128.0f ? -128.0f : (q > 127.0f ? 127.0f : q);
        x[e] = q * scale;
    }
}

// zero_centred_norm (GAIN: ops.rs:44-50) or unit_rms (ops.rs:60-66) of v [n]
// in LDS, then fake_quantise_int8 (ops.rs:120-125), then prepare and the codes
// (n3_codes_from), without writing the normalised vector: one pass computes
// the squares for the eight chains of ops.rs:7-17 and the peak of m_i = (1 +
// gain_i) * v_i (v_i without the gain); since rounding is monotone, the peak
// of the normalised m_i * inverse is fl(peak_m * inverse) exactly, so the
// quantisation scale is known when the inverse is. v and gain 16-byte aligned,
// n a multiple of 32 (the eight chains' squares four a read), sq LDS scratch of
// n + 64 floats, red of at least 32.
template <bool GAIN>
__device__ void n3_norm_codes(const float* v, const float* gain, int n, float* red, float* sq, int P, int group,
                              float wht_scale, int ib, int4* xq, float* xs) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, waves = blockDim.x >> 6, n8 = n / 8;
    const int stride = n8 + 8;
    float pk = 0.0f;
    for (int i = tid; i < n; i += blockDim.x) {
        const float x = v[i];
        sq[(i & 7) * stride + (i >> 3)] = x * x;
        pk = fmaxf(pk, fabsf(GAIN ? (1.0f + gain[i]) * x : x));
    }
    pk = wave_max(pk);
    if (lane == 0) red[16 + wave] = pk;
    __syncthreads();
    if (tid < 8) {
        red[tid] = n3_chain4(reinterpret_cast<const float4*>(sq + tid * stride), n8 / 4);
    }
    __syncthreads();
    float total = 0.0f;
    for (int j = 0; j < 8; ++j) total = total + red[j];
    const float inverse = reciprocal(sqrtf(total / (float)n + 1e-6f));
    float r = red[16 + min(lane, waves - 1)];
    r = fmaxf(r, lane_xor<1>(r));
    r = fmaxf(r, lane_xor<2>(r));
    r = fmaxf(r, lane_xor<4>(r));
    r = fmaxf(r, lane_xor<8>(r));
    const float scale = int8_scale_from_peak(lane_float(r, 0) * inverse);
    n3_codes_from(
        [&](int L, float (&x)[4]) {
            const float4 t = reinterpret_cast<const float4*>(v)[L];
            x[0] = t.x;
            x[1] = t.y;
            x[2] = t.z;
            x[3] = t.w;
            if (GAIN) {
                const float4 g = reinterpret_cast<const float4*>(gain)[L];
                x[0] = (1.0f + g.x) * x[0];
                x[1] = (1.0f + g.y) * x[1];
                x[2] = (1.0f + g.z) * x[2];
                x[3] = (1.0f + g.w) * x[3];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = 4 * L + e < n ? x[e] * inverse : 0.0f;  // fake quantised: still zero
            n3_fake_quantise4(x, scale);
        },
        P, group, wht_scale, ib, xq, xs);
}

// Per-group int8 codes of an LDS input (panel.rs:52-66): scale = peak / 127 (1
// for a zero peak), code = round-half-even(v / scale) clamped. A lane per run
// of 16; the group's peak over its aligned lanes. Codes are stored in the
// order the packed indices decode: for 2-bit dword k of a run holds elements
// k, 4+k, 8+k, 12+k; for 4-bit dword 2h+k holds 8h+k, 8h+2+k, 8h+4+k, 8h+6+k.
__device__ void n3_group_codes(const float* v, int P, int group, int ib, int4* xq, float* xs) {
    const int runs = P / 16, rpg = group / 16;
    for (int base = 0; base < runs; base += blockDim.x) {
        const int u = base + threadIdx.x;
        const bool valid = u < runs;
        float x[16];
        float peak = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            x[i] = valid ? v[16 * u + i] : 0.0f;
            peak = fmaxf(peak, fabsf(x[i]));
        }
        for (int m = 1; m < rpg; m <<= 1) peak = fmaxf(peak, __shfl_xor(peak, m, 64));
        const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
        int c[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) c[i] = quantise_one(x[i], scale);
        if (valid) {
            xq[u] = ib == 2 ? make_int4(n3_b4(c[0], c[4], c[8], c[12]), n3_b4(c[1], c[5], c[9], c[13]),
                                        n3_b4(c[2], c[6], c[10], c[14]), n3_b4(c[3], c[7], c[11], c[15]))
                            : make_int4(n3_b4(c[0], c[2], c[4], c[6]), n3_b4(c[1], c[3], c[5], c[7]),
                                        n3_b4(c[8], c[10], c[12], c[14]), n3_b4(c[9], c[11], c[13], c[15]));
            if (u % rpg == 0) xs[u / rpg] = scale;
        }
    }
    __syncthreads();
}

// Rows row_of(0..R) of a codebook matrix into LDS: the packed bytes (R x
// row_bytes, row r at r * row_bytes) and the fp16 norms (R x groups). Four
// 16-byte loads a thread are issued before their stores.
template <typename RowOf>
__device__ void n3_stage_rows(const CodebookParams& c, RowOf row_of, int R, uint8_t* w, uint16_t* nm) {
    const int chunks = c.row_bytes / 16, total = R * chunks;
    for (int base = 0; base < total; base += 4 * blockDim.x) {
        int4 t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = base + j * blockDim.x + threadIdx.x;
            if (i < total) {
                const int r = i / chunks, k = i - r * chunks;
                t[j] = reinterpret_cast<const int4*>(c.packed + (size_t)row_of(r) * c.row_bytes)[k];
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = base + j * blockDim.x + threadIdx.x;
            if (i < total) reinterpret_cast<int4*>(w)[i] = t[j];
        }
    }
    const int G = c.padded / c.group;
    for (int i = threadIdx.x; i < R * G; i += blockDim.x) {
        const int r = i / G;
        nm[i] = c.norms[(size_t)row_of(r) * G + (i - r * G)];
    }
}

// The integer path of a codebook matrix (panel.rs:153-197 for 2-bit,
// neon.rs:126-183 for 4-bit and ternary) over R rows staged in LDS (w, nm) for
// one input quantised per group in LDS (xq, xs): exact group sums of level *
// code, then per row the epilogue over the groups in order. Lane l of every
// wave holds the codes of run u = l (+ 64 per pass) in registers; the waves
// take the rows in turn, KR at a time. A group's runs sit on aligned lanes
// and join by DPP. No branch inside the loops but uniform ones: groups past
// the row's last add an exact zero (level, norm and scale all zero).
template <int IB, int KR, bool LDS = false>
__device__ void n3_rows_ib(const CodebookParams& c, const uint8_t* w, const uint16_t* nm, int R, const int4* xq,
                           const float* xs, int* acc, float* y) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const int runs = c.padded / 16, rpg = c.group / 16, G = c.padded / c.group;
    const int rpg_shift = rpg == 4 ? 2 : (rpg == 8 ? 3 : 4);
    const uint32_t lut[4] = {c.lut[0], c.lut[1], c.lut[2], c.lut[3]};
    for (int u0 = 0; u0 < runs; u0 += 64) {
        const int u = u0 + lane;
        const bool live = u < runs;
        int4 x = xq[min(u, runs - 1)];
        if (!live) x = make_int4(0, 0, 0, 0);
        const uint8_t* base = w + (size_t)min(u, runs - 1) * 2 * IB;
        const bool leader = live && (u & (rpg - 1)) == 0;
        for (int r0 = wave; r0 < R; r0 += KR * waves) {
            // the KR rows' words first (rows past R repeat the last; a lane past
            // the runs has zero codes, so its sums are zero), then the sums
            int sum[KR];
            if constexpr (IB == 2) {
                uint32_t wd[KR];
#pragma unroll
                for (int k = 0; k < KR; ++k)
                    wd[k] = *reinterpret_cast<const uint32_t*>(base + (size_t)min(r0 + k * waves, R - 1) * c.row_bytes);
#pragma unroll
                for (int k = 0; k < KR; ++k) {
                    int sm = dot4(n3_decode4<2>(wd[k] & 0x03030303u, lut), x.x, 0);
                    sm = dot4(n3_decode4<2>((wd[k] >> 2) & 0x03030303u, lut), x.y, sm);
                    sm = dot4(n3_decode4<2>((wd[k] >> 4) & 0x03030303u, lut), x.z, sm);
                    sum[k] = dot4(n3_decode4<2>((wd[k] >> 6) & 0x03030303u, lut), x.w, sm);
                }
            } else {
                uint2 wd[KR];
#pragma unroll
                for (int k = 0; k < KR; ++k)
                    wd[k] = *reinterpret_cast<const uint2*>(base + (size_t)min(r0 + k * waves, R - 1) * c.row_bytes);
#pragma unroll
                for (int k = 0; k < KR; ++k) {
                    int sm = dot4(n3_decode4<4>(wd[k].x & 0x0f0f0f0fu, lut), x.x, 0);
                    sm = dot4(n3_decode4<4>((wd[k].x >> 4) & 0x0f0f0f0fu, lut), x.y, sm);
                    sm = dot4(n3_decode4<4>(wd[k].y & 0x0f0f0f0fu, lut), x.z, sm);
                    sum[k] = dot4(n3_decode4<4>((wd[k].y >> 4) & 0x0f0f0f0fu, lut), x.w, sm);
                }
            }
#pragma unroll
            for (int k = 0; k < KR; ++k) {
                int v = sum[k];
                v = v + dpp_move<0xb1>(v);
                v = v + dpp_move<0x4e>(v);
                const int v8 = dpp_move<0x141>(v);
                v = rpg >= 8 ? v + v8 : v;
                const int v16 = dpp_move<0x140>(v);
                v = rpg >= 16 ? v + v16 : v;
                sum[k] = v;
            }
#pragma unroll
            for (int k = 0; k < KR; ++k) {
                const int r = r0 + k * waves;
                if (leader && r < R) acc[r * G + (u >> rpg_shift)] = sum[k];
            }
        }
    }
    if constexpr (LDS) lds_barrier(); else __syncthreads();
    const bool fma_form = c.bits == 2;  // panel.rs:184-188; else neon.rs:158,180
    const float lscale = c.lscale;
    for (int r = threadIdx.x; r < R; r += blockDim.x) {
        float t = 0.0f;
        for (int g0 = 0; g0 < G; g0 += 8) {
            float nv[8], av[8], sv[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                // loaded unconditionally (clamped), then zeroed past the
                // groups: a conditional load becomes a branch with its own wait
                const int g = min(g0 + k, G - 1);
                const bool in = g0 + k < G;
                const float n_raw = __half2float(__ushort_as_half(nm[r * G + g]));
                const float a_raw = (float)acc[r * G + g], s_raw = xs[g];
                nv[k] = in ? n_raw : 0.0f;
                av[k] = in ? a_raw : 0.0f;
                sv[k] = in ? s_raw : 0.0f;
            }
            if (fma_form) {
#pragma unroll
                for (int k = 0; k < 8; ++k) t = fmaf(av[k], (nv[k] * lscale) * sv[k], t);
            } else {
#pragma unroll
                for (int k = 0; k < 8; ++k) t = t + (((av[k] * nv[k]) * lscale) * sv[k]);
            }
        }
        y[r] = t;
    }
    if constexpr (LDS) lds_barrier(); else __syncthreads();
}

template <int IB, bool LDS>
__device__ __forceinline__ void n3_rows_kr(const CodebookParams& c, const uint8_t* w, const uint16_t* nm, int R,
                                           const int4* xq, const float* xs, int* acc, float* y) {
    const int waves = blockDim.x >> 6, kr = (R + waves - 1) / waves;
    if (kr <= 1)
        n3_rows_ib<IB, 1, LDS>(c, w, nm, R, xq, xs, acc, y);
    else if (kr <= 2)
        n3_rows_ib<IB, 2, LDS>(c, w, nm, R, xq, xs, acc, y);
    else
        n3_rows_ib<IB, 4, LDS>(c, w, nm, R, xq, xs, acc, y);
}

// LDS: the barriers wait for LDS operations only (w, nm, xq, xs, acc and y in
// LDS, or y in memory that no thread of the block reads back).
template <bool LDS = false>
__device__ void n3_rows(const CodebookParams& c, const uint8_t* w, const uint16_t* nm, int R, const int4* xq,
                        const float* xs, int* acc, float* y) {
    if (c.bits == 4)
        n3_rows_kr<4, LDS>(c, w, nm, R, xq, xs, acc, y);
    else
        n3_rows_kr<2, LDS>(c, w, nm, R, xq, xs, acc, y);
}

struct N3AttentionParams {
    CodebookParams qkvg;       // rows q [H*64] | k [KV*64] | v [KV*64] | gate [H*64]
    const int4* codes;         // [padded / 16] the projections' input, prepared and quantised (plane order)
    const float* code_scales;  // [groups]
    float* hist;               // conv-tap ring [taps][q | k | v]
    const float* taps[3];
    int ntaps, position, H, KV, cap, first, count;
    const float* q_norm;
    const float* k_norm;
    const float* cos_row;
    const float* sin_row;
    int8_t* keys;
    float* key_scales;
    int8_t* values;
    float* value_scales;
    float* out;  // [H][64], times sigmoid(gate)
};

constexpr int kN3AttendThreads = 1024;
constexpr int kN3StagedPositions = 1024;  // earlier positions whose keys and values the attention block holds
constexpr int kN3HeadRowBytes = 256;  // the head's 256 staged rows, each at most 256 bytes (2-bit, 1024 columns)
constexpr int kN3MaxTaps = 4;

// One block a query head (attention.rs:96-149 for that head): every load this
// block needs is issued first (its 256 projection rows and norms, the input
// codes, the conv taps and ring samples, the norm gains and rotary row, and
// the cached keys and values of the earlier positions, which no block writes
// here); the new position's key and value come from LDS. Its threads share
// data through LDS only (the cache rows and ring samples it stores are not read
// back), so its barriers wait for LDS operations and leave global loads (the
// staged values' LDS copies included, which each wave waits for itself before
// the barrier that publishes them) in flight.
__global__ __launch_bounds__(kN3AttendThreads) void n3_attention_kernel(N3AttentionParams p) {
    __shared__ __align__(16) uint8_t w_s[256 * kN3HeadRowBytes];
    __shared__ uint16_t nm_s[256 * 16];
    __shared__ int4 xq[kN3Hadamard / 16];
    __shared__ float xs[64];
    __shared__ int acc[64 * kN3Head];  // the row group sums, then the value sums
    __shared__ float y_s[256];
    __shared__ float v_s[3][kN3Head];
    __shared__ float red_s[3][8];
    __shared__ __align__(16) int8_t qc_s[kN3Head];
    __shared__ __align__(16) int8_t kc_s[kN3Head];
    __shared__ __align__(16) int8_t vc_s[kN3Head];
    __shared__ float scale_s[3];
    __shared__ float c_s[kN3MaxAttend];
    __shared__ float red[16];
    __shared__ float lanes_s[4];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int group = p.H / p.KV, kvh = h / group, P = p.qkvg.padded, G = P / p.qkvg.group;
    const int qw = p.H * kN3Head, kw = p.KV * kN3Head, width_all = qw + 2 * kw;
    const int count = p.count, last = count - 1;  // the new position is first + last
    // ---- loads: none conditional (indices clamped), so that the values stay in
    // registers and every request is out before the first wait. The head's rows
    // are four ranges of 64 (q rows, its kv head's k and v rows, gate rows),
    // staged one after another.
    const int chunks = p.qkvg.row_bytes / 16, per_range = 64 * chunks;
    // the first row of range rj: uniform steps added per lane (neither a branch
    // nor a lookup table in memory)
    const int row0 = h * 64, step1 = qw + kvh * 64 - row0, step2 = kw, step3 = kw + (h - kvh) * 64;
    auto range_row = [&](int rj) {
        return row0 + (rj >= 1 ? step1 : 0) + (rj >= 2 ? step2 : 0) + (rj >= 3 ? step3 : 0);
    };
    int4 rw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = min(j * kN3AttendThreads + tid, 4 * per_range - 1);
        const int rj = (i >= per_range) + (i >= 2 * per_range) + (i >= 3 * per_range);
        rw[j] = reinterpret_cast<const int4*>(p.qkvg.packed + (size_t)range_row(rj) * p.qkvg.row_bytes)[i - rj * per_range];
    }
    uint16_t rn[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = min(j * kN3AttendThreads + tid, 256 * G - 1), per = 64 * G;
        const int rj = (i >= per) + (i >= 2 * per) + (i >= 3 * per);
        rn[j] = p.qkvg.norms[(size_t)range_row(rj) * G + (i - rj * per)];
    }
    // (the small inputs below are requested by the waves that use them only:
    // every 16-byte request of a wave takes the CU's load path whether or not
    // its lanes share an address)
    int4 code_any = make_int4(0, 0, 0, 0);
    float code_scale_any = 0.0f;
    if (wave == 0) {
        code_any = p.codes[min(tid, P / 16 - 1)];
        code_scale_any = p.code_scales[min(tid, G - 1)];
    }
    // conv taps, ring samples, norm gain and rotary row of waves 0, 1, 2 (q, k, v)
    const int which = wave < 3 ? wave : 0;
    const int head = which == 0 ? h : kvh;
    const int width = which == 0 ? qw : kw, off = which == 0 ? 0 : (which == 1 ? qw : qw + kw);
    const int col = head * kN3Head + lane;
    // (every wave requests them, from indices that exist: with no taps the
    // loads read the norm gains instead and are not used; a load under a
    // condition would be sunk into a branch and waited for there)
    const bool has_taps = p.ntaps > 0;
    const int ntap = has_taps ? min(p.ntaps, p.position + 1) : 0;
    const float* const tap = !has_taps ? p.q_norm : which == 0 ? p.taps[0] : which == 1 ? p.taps[1] : p.taps[2];
    const float* const ring = has_taps ? p.hist : p.q_norm;
    float gains[kN3MaxTaps], samples[kN3MaxTaps];  // set and used by waves 0..2
    // the norm gain and rotary row (used by waves 0 and 1): every wave
    // requests them, unconditionally (a value chosen by a branch would bring
    // the 1 + gain of its use into the branch, and its wait with it)
    const float gain = (which == 0 ? p.q_norm : p.k_norm)[lane];
    const float cs = p.cos_row[lane & 31], sn = p.sin_row[lane & 31];
    if (wave < 3) {
#pragma unroll
        for (int t = 0; t < kN3MaxTaps; ++t) {
            const int tc = has_taps ? min(t, ntap - 1) : 0;
            const float g = tap[has_taps ? (size_t)tc * width + col : (size_t)lane];
            const float sm = ring[has_taps ? (size_t)((p.position - tc) % p.ntaps) * width_all + off + col : (size_t)lane];
            gains[t] = g;    // used for t < ntap only
            samples[t] = sm;  // used for 1 <= t < ntap only
        }
    }
    // the first 1024 earlier positions' keys and values as 16-byte units (unit u
    // = 1024 k + tid: quarter u % 4 of position u / 4, so a wave's request is 1
    // KB in a row and a position's four quarters sit on one quad), and each
    // unit's key scale; thread t's value scale of position t. A unit past the
    // earlier positions reads the last of them, or the new position's row when
    // there is none, and is not used. Later positions are read from memory as
    // they are needed.
    const int8_t* kbase = p.keys + ((size_t)kvh * p.cap + p.first) * kN3Head;
    const int8_t* vbase = p.values + ((size_t)kvh * p.cap + p.first) * kN3Head;
    const float* ks = p.key_scales + (size_t)kvh * p.cap + p.first;
    const float* vsc = p.value_scales + (size_t)kvh * p.cap + p.first;
    const int early = min(last, kN3StagedPositions), clampp = max(last - 1, 0);
    // ---- the head's projection rows (stored unconditionally: every index is
    // inside w_s and nm_s, and units past the rows hold clamped copies that
    // are never read; a store under a condition takes its load into a branch
    // that waits for it alone)
    static_assert(4 * kN3AttendThreads * 16 <= sizeof(w_s) && 4 * kN3AttendThreads <= 256 * 16, "staging fits");
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = j * kN3AttendThreads + tid;
        reinterpret_cast<int4*>(w_s)[i] = rw[j];
        nm_s[i] = rn[j];
    }
    if (tid < P / 16) xq[tid] = code_any;
    if (tid < G) xs[tid] = code_scale_any;
    // the keys are requested after the staged rows arrive (a wait counts
    // loads in issue order: keys requested first would delay the rows), and
    // stream in during the row products
    int4 ku[4];
    float ksr[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int u = k * kN3AttendThreads + tid, pos = min(u >> 2, clampp);
        ku[k] = reinterpret_cast<const int4*>(kbase + (size_t)pos * kN3Head)[u & 3];
        ksr[k] = ks[pos];
    }
    lds_barrier();
    n3_rows<true>(p.qkvg, w_s, nm_s, 256, xq, xs, acc, y_s);
    // the rows are done: the values of the staged positions are requested now
    // (they arrive during the next phases; w_s then takes them, [position][64],
    // and nm_s their scales)
    int8_t* const val_s = reinterpret_cast<int8_t*>(w_s);
    float* const vsc_s = reinterpret_cast<float*>(nm_s);
    {  // global_load_lds: wave w copies 1 KB chunks w, w + 16, ... (lane l: unit 64 c + l)
        const int units = 4 * early, wv = __builtin_amdgcn_readfirstlane(wave);
        for (int c = wv; c < (units + 63) / 64; c += kN3AttendThreads / 64)
            if (64 * c + lane < units)
                __builtin_amdgcn_global_load_lds((n3_global_void*)(vbase + (size_t)(64 * c + lane) * 16),
                                                 (n3_lds_void*)(val_s + (size_t)c * 1024), 16, 0, 0);
    }
    const float vsr = vsc[min(tid, clampp)];
    // ---- conv taps, norms, rotary, codes (attention.rs:110-141)
    float v = 0.0f;
    if (wave < 3) {
        const float raw = y_s[which * 64 + lane];
        v = raw;
        if (p.ntaps > 0) {
            p.hist[(size_t)(p.position % p.ntaps) * width_all + off + col] = raw;
            v = 0.0f;
#pragma unroll
            for (int t = 0; t < kN3MaxTaps; ++t)
                if (t < ntap) v = v + gains[t] * (t == 0 ? raw : samples[t]);
        }
        v_s[which][lane] = v;
    }
    lds_barrier();
    if (wave < 2 && lane < 8) {
        float s = 0.0f;
        for (int c = 0; c < kN3Head / 8; ++c) s = s + v_s[which][8 * c + lane] * v_s[which][8 * c + lane];
        red_s[which][lane] = s;
    }
    lds_barrier();
    if (wave < 2) {
        float ss = 0.0f;
        for (int j = 0; j < 8; ++j) ss = ss + red_s[which][j];
        const float inverse = reciprocal(sqrtf(ss / (float)kN3Head + 1e-6f));
        v = ((1.0f + gain) * v) * inverse;
    }
    lds_barrier();
    if (wave < 2) v_s[which][lane] = v;
    lds_barrier();
    if (wave < 2) {
        const int half = kN3Head / 2;
        if (lane < half) {
            const float a = v_s[which][lane], bb = v_s[which][lane + half];
            v = a * cs - bb * sn;
        } else {
            const float a = v_s[which][lane - half], bb = v_s[which][lane];
            v = bb * cs + a * sn;
        }
    }
    if (wave < 3) {  // ops.rs:112-118 per head
        const float peak = wave_max(fabsf(v));
        const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
        const int8_t code8 = (int8_t)quantise_one(v, scale);
        (which == 0 ? qc_s : which == 1 ? kc_s : vc_s)[lane] = code8;
        if (lane == 0) scale_s[which] = scale;
        if (which > 0) {  // the cache append (the blocks of a kv group write the same bytes)
            const size_t row = (size_t)kvh * p.cap + p.position;
            (which == 1 ? p.keys : p.values)[row * kN3Head + lane] = code8;
            if (lane == 0) (which == 1 ? p.key_scales : p.value_scales)[row] = scale;
        }
    }
    lds_barrier();
    // ---- kernels/src/attention.rs:53-80 (as n3_attend_kernel)
    const float query_scale = scale_s[0] * (1.0f / sqrtf((float)kN3Head));
    float peak = -INFINITY;
    {  // the staged positions: a quad a position, each lane one quarter's dot
        const int4 qq = reinterpret_cast<const int4*>(qc_s)[tid & 3];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int u = k * kN3AttendThreads + tid, pos = u >> 2;
            int sc = dot16(qq, ku[k], 0);
            sc = sc + dpp_move<0xb1>(sc);
            sc = sc + dpp_move<0x4e>(sc);
            if (pos < early) {
                const float c = ((float)sc * ksr[k]) * query_scale;
                if ((u & 3) == 0) c_s[pos] = c;
                peak = fmaxf(peak, c);
            }
        }
    }
    // the new position, and earlier positions past the staged ones
    for (int pp = early + tid; pp < count; pp += kN3AttendThreads) {
        // the new position's key from LDS, another's from memory (values
        // selected, so that no load is a flat one)
        int4 k[4];
        float kscl = scale_s[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) k[i] = reinterpret_cast<const int4*>(kc_s)[i];
        if (pp != last) {
#pragma unroll
            for (int i = 0; i < 4; ++i) k[i] = reinterpret_cast<const int4*>(kbase + (size_t)pp * kN3Head)[i];
            kscl = ks[pp];
        }
        int score = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) score = dot16(reinterpret_cast<const int4*>(qc_s)[i], k[i], score);
        const float c = ((float)score * kscl) * query_scale;
        c_s[pp] = c;
        peak = fmaxf(peak, c);
    }
    peak = n3_block_max<true, true>(peak, red);
    // (a thread's first position is its own: its value scale is in vsr)
    auto value_scale = [&](int pp) {
        return pp == last ? scale_s[2] : pp == tid ? vsr : pp < early ? vsc_s[pp] : vsc[pp];
    };
    float cpeak = 0.0f;
    for (int pp = tid; pp < count; pp += kN3AttendThreads) {
        const float e = fast_exp(c_s[pp] - peak);
        c_s[pp] = e;
        cpeak = fmaxf(cpeak, fabsf(e * value_scale(pp)));
    }
    if (tid < early) vsc_s[tid] = vsr;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's value chunks are in LDS (published by the barriers below)
    cpeak = n3_block_max<true, true>(cpeak, red);
    // the coefficients round((e * value scale) / scale), once a position
    // (quotients<1>: rounds as the division; in acc, free until the sums)
    const float scale = cpeak / 2047.0f;
    int* const wgt_s = acc;
    const bool pre_w = count <= 64 * kN3Head;
    if (pre_w && cpeak > 0.0f) {
        for (int pp = tid; pp < count; pp += kN3AttendThreads) {
            const float x = c_s[pp] * value_scale(pp);
            float y;
            quotients<1>(&x, scale, &y);
            wgt_s[pp] = (int)__builtin_roundf(y);
        }
    }
    lds_barrier();
    const int vector_count = count - count % 4;
    if (tid < 4) {
        float s = 0.0f;
        int pp = tid;
        for (; pp + 64 <= vector_count; pp += 64) {
            float e[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) e[j] = c_s[pp + 4 * j];
#pragma unroll
            for (int j = 0; j < 16; ++j) s = s + e[j];
        }
        for (; pp < vector_count; pp += 4) s = s + c_s[pp];
        lanes_s[tid] = s;
    }
    // the value sums: thread (dg, pc) takes dims 4 dg .. 4 dg + 3 of positions
    // pc, pc + 64, ... (integer sums: any order)
    const int dg = tid & 15, pc = tid >> 4;
    int av[4] = {0, 0, 0, 0};
    if (cpeak > 0.0f) {
        for (int pp0 = pc; pp0 < count; pp0 += 16 * 64) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int pp = pp0 + 64 * j;
                if (pp >= count) break;
                // staged and new values read as LDS (values selected, not
                // addresses, so that no load is a flat one); a later earlier
                // position (past the staged ones) from memory
                const int staged = reinterpret_cast<const int*>(val_s + (size_t)min(pp, kN3StagedPositions - 1) * kN3Head)[dg];
                const int fresh = reinterpret_cast<const int*>(vc_s)[dg];
                int packed = pp == last ? fresh : staged;
                if (pp >= early && pp != last) packed = *reinterpret_cast<const int*>(vbase + (size_t)pp * kN3Head + 4 * dg);
                const int wgt = pre_w ? wgt_s[pp] : (int)__builtin_roundf((c_s[pp] * value_scale(pp)) / scale);
#pragma unroll
                for (int k = 0; k < 4; ++k) av[k] += wgt * (int)(int8_t)(packed >> (8 * k));
            }
        }
    }
    lds_barrier();  // the coefficients are read: acc takes the sums
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[pc * kN3Head + 4 * dg + k] = av[k];
    lds_barrier();
    if (tid < kN3Head) {
        int sum = 0;
        for (int c = 0; c < 64; ++c) sum += acc[c * kN3Head + tid];
        float total = (lanes_s[0] + lanes_s[1]) + (lanes_s[2] + lanes_s[3]);
        for (int pp = vector_count; pp < count; ++pp) total = total + c_s[pp];
        float o = cpeak > 0.0f ? (float)sum * scale : 0.0f;
        o = o * reciprocal(total);
        o = o * libm_sigmoid(y_s[192 + tid]);
        p.out[(size_t)h * kN3Head + tid] = o;
    }
}

struct N3OutParams {
    CodebookParams out;
    const float* attended;  // [n] gated attention
    int n;
    float* y;               // [rows]
};

constexpr int kN3OutRowBytes = 1024;  // 4-bit over 2048 columns or 2-bit over 4096

// fake_quantise_int8 of the gated attention, prepare, then rows
// [64 * blockIdx.x, + 64) of the output projection (attention.rs:150-153).
// The block's rows, norms and the attention are requested together first.
template <int LPT>
__global__ __launch_bounds__(1024) void n3_out_kernel(N3OutParams p) {
    __shared__ __align__(16) uint8_t w_s[64 * kN3OutRowBytes];
    __shared__ __align__(16) uint16_t nm_s[64 * 64 + 8];
    __shared__ __align__(16) float v[kN3MaxWidth];
    __shared__ int4 xq[kN3MaxWidth / 16];
    __shared__ float xs[64];
    __shared__ int acc[64 * 64];
    __shared__ float y_s[64];
    __shared__ float red[16];
    constexpr int T = 1024;
    const int P = p.out.padded, G = P / p.out.group, tid = threadIdx.x;
    const int r0 = blockIdx.x * 64, R = min(64, p.out.rows - r0);
    // the block's rows are contiguous: LPT 16-byte loads a thread, then the
    // norms and the input vector, none conditional (indices clamped; the last
    // norm unit may run into the next rows' norms or the blob's padding)
    const int units = R * (p.out.row_bytes / 16);
    const int4* wsrc = reinterpret_cast<const int4*>(p.out.packed + (size_t)r0 * p.out.row_bytes);
    int4 rw[LPT];
#pragma unroll
    for (int j = 0; j < LPT; ++j) rw[j] = wsrc[min(j * T + tid, units - 1)];
    const int nn = (R * G * 2 + 15) / 16, n4 = p.n / 4;
    const int4 rn = reinterpret_cast<const int4*>(p.out.norms + (size_t)r0 * G)[min(tid, nn - 1)];
    const float4 a = reinterpret_cast<const float4*>(p.attended)[min(tid, n4 - 1)];
#pragma unroll
    for (int j = 0; j < LPT; ++j)
        if (j * T + tid < units) reinterpret_cast<int4*>(w_s)[j * T + tid] = rw[j];
    if (tid < nn) reinterpret_cast<int4*>(nm_s)[tid] = rn;
    if (tid < n4) reinterpret_cast<float4*>(v)[tid] = a;
    // the peak of the attention from the registers (ops.rs:32-43, order-free)
    {
        float pk = tid < n4 ? fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))) : 0.0f;
        pk = wave_max(pk);
        if ((tid & 63) == 0) red[tid >> 6] = pk;
    }
    __syncthreads();
    // fake_quantise_int8 (ops.rs:120-125) as the values are loaded for prepare and the codes
    float peak = red[min(tid & 63, T / 64 - 1)];
    peak = fmaxf(peak, lane_xor<1>(peak));
    peak = fmaxf(peak, lane_xor<2>(peak));
    peak = fmaxf(peak, lane_xor<4>(peak));
    peak = fmaxf(peak, lane_xor<8>(peak));
    const float scale = int8_scale_from_peak(lane_float(peak, 0));
    const int n = p.n;
    n3_codes_from(
        [&](int L, float (&x)[4]) {
            const float4 t = reinterpret_cast<const float4*>(v)[L];
            x[0] = 4 * L < n ? t.x : 0.0f;
            x[1] = 4 * L + 1 < n ? t.y : 0.0f;
            x[2] = 4 * L + 2 < n ? t.z : 0.0f;
            x[3] = 4 * L + 3 < n ? t.w : 0.0f;
            n3_fake_quantise4(x, scale);
        },
        P, p.out.group, p.out.wht_scale, p.out.bits == 5 ? 2 : p.out.bits, xq, xs);
    __syncthreads();
    n3_rows(p.out, w_s, nm_s, R, xq, xs, acc, y_s);
    if (tid < R) p.y[r0 + tid] = y_s[tid];
}

struct N3BoundaryParams {
    int tail, final, route;
    N3BlockOutParams t;          // the tail of the previous layer
    const float* final_norm;
    float* hidden;
    // the routing of layer `layer` at `slot` (lanes.rs:48-84)
    int layer, slot;
    const float* stream;         // when there is no tail: the lanes stream
    CodebookParams phi_pre, phi_post, phi_res;
    const float *a_pre, *a_post, *a_res, *b_pre, *b_post, *b_res;
    float* input;                // [d]
    float* post;                 // [lanes]
    float* residual;             // [lanes][lanes]
    // the block input (session.rs:112-118)
    const float* key;
    const float* value;
    const float* norm_in;
    float* x;
    int qpadded, qgroup, qib;
    float qscale;
    int4* codes;          // [qpadded / 16] the projections' input, prepared and quantised
    float* code_scales;   // [qpadded / qgroup]
    const uint8_t* phi_rows;  // the route layer's rows of phi_pre, phi_post, phi_res, one after another
    int d, lanes;
    // a run of tokens, one block each (prefill.rs:45-88): block b's vectors
    // sit b strides on (stream and next lanes * d, attention, x, input, key
    // and value d, post kMaxLanes, residual kMaxLanes^2, cell cell_stride,
    // rotated qpadded); with `rotated` the block input is written prepared
    // (matrix.rs:123-128) instead of as codes; the last block writes hidden
    float* rotated;
    int cell_stride;
    // with the final norm: the logits' input (fake_quantise_int8 of the hidden
    // state, then prepare for the embedding matrix: session.rs:151-165) into
    // logits_in [lpadded] as well
    float* logits_in;
    int lpadded, lgroup;
    float lwht;
    // with `raw` (one token at `position`), the engram value is the site's
    // convolution (engram.rs:84-111) of its raw value over the ring, computed
    // here, and the raw value joins the ring (slot position mod keep)
    const float* raw;
    float* ring;
    const float* taps;
    int position, keep, ntaps, dilation;
};

constexpr int kN3RouteRows = 24;         // 2 lanes + lanes^2 for four lanes
constexpr int kN3RouteRowBytes = 768;    // 2-bit over 3072 columns

__global__ __launch_bounds__(kN3Block) void n3_boundary_kernel(N3BoundaryParams p) {
    __shared__ __align__(16) float xs_[kN3Hadamard], a_[kN3Hadamard], sc_[kN3Hadamard], st_[kN3Hadamard], mx_[kN3Hadamard];
    __shared__ float mod_[kN3Hadamard];
    __shared__ float chains_[32];
    __shared__ float weights_[64];
    __shared__ float red[32];
    __shared__ __align__(16) float tailw_s[6 * kN3Hadamard + kN3Hadamard * 8];  // the six factors, then cond_v
    __shared__ __align__(16) float stream_s[kN3MaxWidth];
    __shared__ __align__(16) float rv[kN3MaxWidth];
    __shared__ int4 rq[kN3MaxWidth / 16];
    __shared__ float rs[64];
    __shared__ float ry[kN3RouteRows];
    __shared__ __align__(16) uint8_t pw[kN3RouteRows * kN3RouteRowBytes];
    __shared__ uint16_t pn[kN3RouteRows * 64];
    __shared__ __align__(16) float tin_s[3 * kN3Hadamard];  // the tail's attention, x and input ([3][d])
    __shared__ float lane_s[2 * kMaxLanes + kMaxLanes * kMaxLanes];  // post, residual of the tail
    __shared__ float small_s[4 * kMaxLanes + 2 * 64];  // a_pre a_post a_res (one each), b_pre, b_post, b_res
    __shared__ float gate_s[kMaxLanes];
    __shared__ float alpha_s;
    const int tid = threadIdx.x, d = p.d, L = p.lanes, S = L * d;
    // everything this block reads from memory, requested first
    const int route_rows = 2 * L + L * L, G = p.phi_pre.padded / p.phi_pre.group;
    const int layer = p.layer, chunks = p.phi_pre.row_bytes / 16;
    N3BlockOutParams t = p.t;
    {  // this block's token of a run
        const size_t b = blockIdx.x;
        t.attention += b * d;
        t.x += b * d;
        t.input += b * d;
        t.post += b * kMaxLanes;
        t.residual += b * kMaxLanes * kMaxLanes;
        t.stream += b * S;
        t.next += b * S;
        t.cell += b * p.cell_stride;
    }
    // (the kernel arguments stay as passed: a changed argument struct is copied
    // to scratch memory)
    const size_t tb = blockIdx.x;
    const float* const in_stream = p.stream + tb * S;
    float* const out_input = p.input + tb * d;
    float* const out_post = p.post + tb * kMaxLanes;
    float* const out_residual = p.residual + tb * kMaxLanes * kMaxLanes;
    const float* const e_key = p.key != nullptr ? p.key + tb * d : nullptr;
    const float* const e_value = p.key != nullptr ? p.value + tb * d : nullptr;
    float* const out_x = p.x + tb * d;
    float* const out_rotated = p.rotated != nullptr ? p.rotated + tb * p.qpadded : nullptr;
    N3TailPre pre{};
    const bool cv_staged = p.tail && t.rank == 8;
    float* const cv_ = tailw_s + 6 * kN3Hadamard;
    // The vectors the tail reads first (attention, x and input; the stream)
    // through registers, two 16-byte units a thread; the later-used ranges (the
    // factors and cond_v, the route layer's rows) go straight to LDS once these
    // are stored, 1 KB a wave instruction, and are waited for before their first
    // use (the condition products, the routing rows), while the tail runs.
    const int u0 = p.tail ? (6 * kN3Hadamard + (cv_staged ? 8 * d : 0)) / 4 : 0, u1 = p.tail ? 3 * d / 4 : 0;
    const int u2 = S / 4, u3 = p.route ? route_rows * chunks : 0, d4 = d / 4;
    // 64-unit chunks, each inside one vector (d a multiple of 256): chunk c of
    // wave c % 16, its source and destination uniform over the wave
    const int cd = d4 / 64, c1 = u1 / 64, cn = (u1 + u2) / 64;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    auto chunk_src = [&](int c) {
        const float* b = c >= c1 ? (p.tail ? t.stream : in_stream) : c < cd ? t.attention : c < 2 * cd ? t.x : t.input;
        const int first = c >= c1 ? c1 : c < cd ? 0 : c < 2 * cd ? cd : 2 * cd;
        return reinterpret_cast<const int4*>(b) + (c - first) * 64;
    };
    auto chunk_dst = [&](int c) {
        return c >= c1 ? reinterpret_cast<int4*>(stream_s) + (c - c1) * 64 : reinterpret_cast<int4*>(tin_s) + c * 64;
    };
    int4 v0 = make_int4(0, 0, 0, 0), v1 = make_int4(0, 0, 0, 0);
    if (wv < cn) v0 = chunk_src(wv)[lane];
    if (wv + 16 < cn) v1 = chunk_src(wv + 16)[lane];
    // the small tensors, one element a thread from a selected address, so
    // that every load is issued before the first wait: the layer's norms of
    // phi_pre, phi_post and phi_res (rows one after another); small_s (a_pre,
    // a_post, a_res, then b_pre, b_post, b_res of the layer); the tail's post
    // and residual
    const int nsmall = 3 + 2 * L + L * L, nlane = L + L * L;
    uint16_t tn = 0;
    float small_v = 0.0f, lane_v = 0.0f;
    if (p.route) {
        const int i = min(tid, route_rows * G - 1), r = i / G;
        const uint16_t* nsrc = r < L ? p.phi_pre.norms + (size_t)(layer * L + r) * G
                                     : r < 2 * L ? p.phi_post.norms + (size_t)(layer * L + r - L) * G
                                                 : p.phi_res.norms + (size_t)(layer * L * L + r - 2 * L) * G;
        tn = nsrc[i - r * G];
        const int j = min(tid, nsmall - 1);
        const float* ssrc = j == 0 ? p.a_pre + layer
                          : j == 1 ? p.a_post + layer
                          : j == 2 ? p.a_res + layer
                          : j < 3 + L ? p.b_pre + layer * L + (j - 3)
                          : j < 3 + 2 * L ? p.b_post + layer * L + (j - 3 - L)
                                          : p.b_res + layer * L * L + (j - 3 - 2 * L);
        small_v = *ssrc;
    }
    if (p.tail) {
        const int j = min(tid, nlane - 1);
        lane_v = *(j < L ? t.post + j : t.residual + (j - L));
        pre = n3_tail_prefetch(t);
    }
    if (p.route && tid < route_rows * G) pn[tid] = tn;
    if (p.route && tid < nsmall) small_s[tid] = small_v;
    if (p.tail && tid < nlane) lane_s[tid < L ? tid : kMaxLanes + tid - L] = lane_v;
    if (wv < cn) chunk_dst(wv)[lane] = v0;
    if (wv + 16 < cn) chunk_dst(wv + 16)[lane] = v1;
    {
        const int c0 = (u0 + 63) / 64, c3 = (u3 + 63) / 64;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
        for (int ch = wave; ch < c0 + c3; ch += kN3Block / 64) {
            const bool first = ch < c0;
            const int k = first ? ch : ch - c0, cnt = first ? u0 : u3;
            const char* src = first ? reinterpret_cast<const char*>(t.factors[0]) : reinterpret_cast<const char*>(p.phi_rows);
            char* dst = first ? reinterpret_cast<char*>(tailw_s) : reinterpret_cast<char*>(pw);
            const int u = 64 * k + lane;
            if (u < cnt)
                __builtin_amdgcn_global_load_lds((n3_global_void*)(src + (size_t)u * 16), (n3_lds_void*)(dst + (size_t)k * 1024),
                                                 16, 0, 0);
        }
    }
    lds_barrier();  // the factors, cond_v and routing rows stay in flight
    const N3TailLds l{xs_, a_, sc_, st_, mx_, mod_, cv_, chains_, weights_, red, tin_s, tailw_s, stream_s, lane_s};
    if (p.tail) n3_tail<true>(t, l, rv, pre);  // the next stream into rv, then into stream_s
    if (p.tail) {
        for (int i = tid; i < S; i += blockDim.x) stream_s[i] = rv[i];
        __syncthreads();
    }
    if (p.final) {  // session.rs:141-144
        for (int i = tid; i < d; i += blockDim.x) {
            float v = 0.0f;
            for (int ln = 0; ln < L; ++ln) v = v + stream_s[(size_t)ln * d + i] / (float)L;
            a_[i] = v;
        }
        __syncthreads();
        n3_norm(a_, p.final_norm, d, a_, red, cv_);
        if (blockIdx.x == gridDim.x - 1)
            for (int i = tid; i < d; i += blockDim.x) p.hidden[i] = a_[i];
        if (p.logits_in != nullptr) {
            n3_fake_quantise(a_, d, red);
            for (int i = d + tid; i < p.lpadded; i += blockDim.x) a_[i] = 0.0f;
            __syncthreads();
            n3_rotate(a_, p.lpadded, p.lgroup, p.lwht);
            if (blockIdx.x == gridDim.x - 1)
                for (int i = tid; i < p.lpadded; i += blockDim.x) p.logits_in[i] = a_[i];
        }
    }
    if (!p.route) return;
    // the block input's tensors, requested before the routing work
    float norm_in_r, key_r, value_r;
    norm_in_r = tid < d ? p.norm_in[tid] : 0.0f;
    key_r = (e_key != nullptr && tid < d) ? e_key[tid] : 0.0f;
    if (p.raw != nullptr) {
        // engram.rs:84-111: value = sum over taps of gain * the raw value
        // `tap * dilation` positions back (the ring holds the earlier ones)
        // (taps of the positions that exist, at most kN3MaxTaps, read first)
        const int i = min(tid, d - 1);
        const float r = p.raw[i];
        // (every load issued unconditionally from a clamped index, then
        // selected: a conditional load becomes a branch with its own wait)
        float gain[kN3MaxTaps], sample[kN3MaxTaps];
        if (p.ntaps > 0) {
#pragma unroll
            for (int tap = 0; tap < kN3MaxTaps; ++tap) {
                const int back = tap * p.dilation;
                const bool on = tap < p.ntaps && p.position >= back;
                const float g_raw = p.taps[(size_t)min(tap, p.ntaps - 1) * d + i];
                const float s_raw = p.ring[(size_t)((on ? p.position - back : p.position) % p.keep) * d + i];
                gain[tap] = on ? g_raw : 0.0f;
                sample[tap] = (on && tap > 0) ? s_raw : r;
            }
        } else {
#pragma unroll
            for (int tap = 0; tap < kN3MaxTaps; ++tap) gain[tap] = sample[tap] = 0.0f;
        }
        float v = 0.0f;
#pragma unroll
        for (int tap = 0; tap < kN3MaxTaps; ++tap)
            if (tap < p.ntaps && p.position >= tap * p.dilation) v = v + gain[tap] * sample[tap];
        if (tid < d) p.ring[(size_t)(p.position % p.keep) * d + i] = r;
        value_r = v;
    } else {
        value_r = (e_key != nullptr && tid < d) ? e_value[tid] : 0.0f;
    }
    // lanes.rs:49-53: unit_rms, fake_quantise_int8, prepare (phi_pre's groups);
    // the routing matrices share their format, so one set of codes serves the
    // three (matrix.rs:167-193 shares a plane input per format)
    const int P = p.phi_pre.padded;
    const int ib_pre = p.phi_pre.bits == 5 ? 2 : p.phi_pre.bits;
    n3_norm_codes<false>(stream_s, nullptr, S, red, cv_, P, p.phi_pre.group, p.phi_pre.wht_scale, ib_pre, rq, rs);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the routing rows, copied into LDS at the start
    __syncthreads();
    // lanes.rs:56-63: the layer's rows of the three routing matrices
    // (the rows' group sums in cv_, free after the tail: R * G <= 1024)
    n3_rows(p.phi_pre, pw, pn, route_rows, rq, rs, reinterpret_cast<int*>(cv_), ry);
    // lanes.rs:64-83 (as lanes_route_kernel)
    const int own = p.slot % L, n = L * L;
    if (tid < 64) {
        if (tid < L) {
            const int lane = tid;
            const float pre_offset = lane == own ? 8.0f + -4.0f : -4.0f;
            gate_s[lane] = libm_sigmoid(small_s[0] * ry[lane] + small_s[3 + lane] + pre_offset);
            const float post_offset = lane == own ? 0.0f : -4.0f;
            out_post[lane] = 2.0f * libm_sigmoid(small_s[1] * ry[L + lane] + small_s[3 + L + lane] + post_offset);
        }
        const int i = tid;
        const bool live = i < n;
        const int r = live ? i / L : 0, c = live ? i % L : 0;
        float m = live ? small_s[2] * ry[2 * L + i] + small_s[3 + 2 * L + i] : 0.0f;
        if (L == 4) {
            // lane 4r + c: a row's entries by quad broadcasts (DPP quad_perm
            // [j,j,j,j]), a column's by rotations of the 16-lane row by 4, 8
            // and 12 (row_ror), each put in row order
            auto row_j = [](float v, int j) {
                const int b = __float_as_int(v);
                const int o = j == 0 ? dpp_move<0x00>(b) : j == 1 ? dpp_move<0x55>(b) : j == 2 ? dpp_move<0xaa>(b)
                                                                                                : dpp_move<0xff>(b);
                return __int_as_float(o);
            };
            // the row each rotation brings, rotated with the values
            const int from4 = dpp_move<0x124>(r), from8 = dpp_move<0x128>(r);
            auto col4 = [&](float v, float (&out)[4]) {
                const int b = __float_as_int(v);
                const float r4 = __int_as_float(dpp_move<0x124>(b)), r8 = __int_as_float(dpp_move<0x128>(b)),
                            r12 = __int_as_float(dpp_move<0x12c>(b));
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    out[j] = j == r ? v : (j == from4 ? r4 : (j == from8 ? r8 : r12));
            };
            float peak = -INFINITY;  // ops.rs:199-202
#pragma unroll
            for (int j = 0; j < 4; ++j) peak = fmaxf(peak, row_j(m, j));
            m = libm_expf(m - peak);
            for (int it = 0; it < 20; ++it) {
                float total = -0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) total = total + row_j(m, j);
                m = m * reciprocal_normal(fmaxf(total, 1.17549435e-38f));
                float col[4];
                col4(m, col);
                total = -0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) total = total + col[j];
                m = m * reciprocal_normal(fmaxf(total, 1.17549435e-38f));
            }
        } else {
            float peak = -INFINITY;
            for (int j = 0; j < L; ++j) peak = fmaxf(peak, __shfl(m, r * L + j, 64));
            m = libm_expf(m - peak);
            for (int it = 0; it < 20; ++it) {
                float total = -0.0f;
                for (int j = 0; j < L; ++j) total = total + __shfl(m, r * L + j, 64);
                m = m * reciprocal_normal(fmaxf(total, 1.17549435e-38f));
                total = -0.0f;
                for (int j = 0; j < L; ++j) total = total + __shfl(m, j * L + c, 64);
                m = m * reciprocal_normal(fmaxf(total, 1.17549435e-38f));
            }
        }
        if (live) out_residual[i] = m;
    }
    __syncthreads();
    for (int i = tid; i < d; i += blockDim.x) {
        float v = 0.0f;
        for (int ln = 0; ln < L; ++ln) v = v + gate_s[ln] * stream_s[(size_t)ln * d + i];
        xs_[i] = v;
        out_input[i] = v;
    }
    __syncthreads();
    // session.rs:112-118 with add_engram (session.rs:175-188)
    if (e_key != nullptr) {
        n3_unit_rms(xs_, d, a_, red, cv_);
        if (tid < d) sc_[tid] = key_r;
        __syncthreads();
        n3_unit_rms(sc_, d, sc_, red, cv_);
        // Iterator::sum: the products by every thread, then in order from -0.0
        if (tid < d) st_[tid] = a_[tid] * sc_[tid];
        __syncthreads();
        if (tid == 0) {
            const float dot = n3_chain4(reinterpret_cast<const float4*>(st_), d / 4, -0.0f);
            alpha_s = libm_sigmoid(dot / sqrtf((float)d));
        }
        __syncthreads();
        const float alpha = alpha_s;
        if (tid < d) xs_[tid] = xs_[tid] + alpha * value_r;
        __syncthreads();
    }
    if (tid < d) mx_[tid] = norm_in_r;
    __syncthreads();
    if (out_rotated != nullptr) {
        n3_norm(xs_, mx_, d, a_, red, cv_);
        n3_fake_quantise(a_, d, red);
        for (int i = d + tid; i < p.qpadded; i += blockDim.x) a_[i] = 0.0f;
        __syncthreads();
        n3_rotate(a_, p.qpadded, p.qgroup, p.qscale);
        for (int i = tid; i < p.qpadded; i += blockDim.x) out_rotated[i] = a_[i];
    } else {
        n3_norm_codes<true>(xs_, mx_, d, red, cv_, p.qpadded, p.qgroup, p.qscale, p.qib, p.codes, p.code_scales);
    }
    for (int i = tid; i < d; i += blockDim.x) out_x[i] = xs_[i];
}

}  // namespace rn

using namespace rn;

// ---- host ---------------------------------------------------------------------

namespace {

int n3_fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return rn::set_error(code, buf);
}

#define N3_HIP(call)                                                                                            \
    do {                                                                                                        \
        hipError_t e_ = (call);                                                                                 \
        if (e_ != hipSuccess)                                                                                   \
            return n3_fail(RN_ERR_DEVICE, "%s: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, __LINE__); \
    } while (0)

#define N3_REQUIRE(cond, ...)                                    \
    do {                                                         \
        if (!(cond)) return n3_fail(RN_ERR_ARGUMENT, __VA_ARGS__); \
    } while (0)

#define N3_CALL(call)               \
    do {                            \
        int rc_ = (call);           \
        if (rc_ != RN_OK) return rc_; \
    } while (0)

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, exponent = (h >> 10) & 0x1f, mantissa = h & 0x3ff;
    uint32_t bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else {  // subnormal: normalise
            int e = -1;
            uint32_t m = mantissa;
            do {
                ++e;
                m <<= 1;
            } while ((m & 0x400) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3ff) << 13);
        }
    } else if (exponent == 31) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 127 - 15) << 23) | (mantissa << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// The canonical tensor order (layout.rs:176-257), walked over the directory.
struct Walk {
    const rn_archive* archive;
    int next = 0, end = 0;
    bool failed = false;
    int take() {
        if (next >= end) {
            failed = true;
            return 0;
        }
        return next++;
    }
    int kind(int index) const {
        rn_tensor_record r;
        return rn_archive_record(archive, index, &r) == RN_OK ? r.kind : 0;
    }
};

}  // namespace

struct N3Layer {
    rn_matrix *q = nullptr, *k = nullptr, *v = nullptr, *gate = nullptr, *out = nullptr;
    rn_matrix* qkvg = nullptr;  // q | k | v | gate rows stacked, when the four share a format
    float *norm_in = nullptr, *q_norm = nullptr, *k_norm = nullptr, *post_norm = nullptr, *pre_norm = nullptr;
    float* taps[3] = {nullptr, nullptr, nullptr};
    float gate_sigmoid = 0.0f;
    float *d1 = nullptr, *d2 = nullptr, *b2 = nullptr, *d3 = nullptr, *d4 = nullptr;
    float* factors[6] = {};
    float *cond_v = nullptr, *cond_u = nullptr;
    int rank = 0;
};

struct N3Engram {
    rn_matrix *tables = nullptr, *key = nullptr, *value = nullptr;
    float* taps = nullptr;
};

struct N3Head {
    int code = 0, layers = 0, per_layer = 0, queries = 0, width = 0;
    float *probes = nullptr, *gain = nullptr, *query = nullptr, *row_bias = nullptr, *bias = nullptr;
    rn_matrix* projection = nullptr;
};

// the bump allocator's state (arena_take)
struct N3Arena {
    char* cur = nullptr;
    size_t left = 0;
};

struct rn_n3_model {
    rn_geometry g{};
    int output_vocab = 0;
    rn_matrix* embedding = nullptr;
    std::vector<N3Layer> layers;
    float *a_pre = nullptr, *a_post = nullptr, *a_res = nullptr, *b_pre = nullptr, *b_post = nullptr,
          *b_res = nullptr;
    std::vector<float> a_pre_h, a_post_h, a_res_h, b_pre_h, b_post_h, b_res_h;
    rn_matrix *phi_pre = nullptr, *phi_post = nullptr, *phi_res = nullptr;
    // the fused step's routing rows by layer, [pre (lanes) | post (lanes) | res
    // (lanes^2)] rows of phi_pre's row bytes each
    uint8_t* phi_stack = nullptr;
    int32_t* perm[2] = {nullptr, nullptr};
    std::vector<N3Engram> engrams;
    float* final_norm = nullptr;
    std::vector<N3Head> heads;
    std::vector<int> active;
    std::vector<void*> allocations;
    N3Arena arena;
    std::vector<rn_matrix*> matrices;
    bool fused = false;  // the three-kernel step applies (integer-path formats, sizes in range)
};

namespace {

// A bump allocator over a few large device allocations, so that the many small
// tensors of a model or a session share pages and address-translation entries
// instead of taking one allocation each. Pieces are 256-byte aligned.
int arena_take(std::vector<void*>& owned, N3Arena& a, size_t bytes, size_t chunk, void** out,
               std::vector<size_t>* sizes = nullptr) {
    bytes = (std::max<size_t>(bytes, 256) + 255) & ~(size_t)255;
    if (bytes > a.left) {
        const size_t size = std::max(chunk, bytes);
        void* p = nullptr;
        N3_HIP(hipMalloc(&p, size));
        owned.push_back(p);
        if (sizes) sizes->push_back(size);
        // a whole chunk starts zeroed (also the part no buffer takes), so that
        // nothing a kernel reads depends on what the memory held before
        // (on the null stream, waited for here: the session streams do not
        // synchronise with it)
        N3_HIP(hipMemset(p, 0, size));
        N3_HIP(hipStreamSynchronize(nullptr));
        a.cur = static_cast<char*>(p);
        a.left = size;
    }
    *out = a.cur;
    a.cur += bytes;
    a.left -= bytes;
    return RN_OK;
}

constexpr size_t kN3ModelChunk = (size_t)8 << 20;
constexpr size_t kN3SessionChunk = (size_t)32 << 20;

int upload_floats(rn_n3_model* m, const std::vector<float>& v, float** out) {
    void* p = nullptr;
    N3_CALL(arena_take(m->allocations, m->arena, v.size() * sizeof(float), kN3ModelChunk, &p));
    if (!v.empty()) N3_HIP(hipMemcpy(p, v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice));
    *out = (float*)p;
    return RN_OK;
}

// tensors.rs:3-13: half or single records as floats
int host_floats(const rn_archive* a, int index, std::vector<float>& out) {
    rn_tensor_record r;
    N3_CALL(rn_archive_record(a, index, &r));
    const uint8_t* data = nullptr;
    size_t n = 0;
    N3_CALL(rn_archive_tensor_bytes(a, index, &data, &n));
    if (r.kind == RN_KIND_HALF) {
        out.resize(n / 2);
        for (size_t i = 0; i < out.size(); ++i) {
            uint16_t h;
            memcpy(&h, data + 2 * i, 2);
            out[i] = half_to_float(h);
        }
    } else if (r.kind == RN_KIND_SINGLE) {
        out.resize(n / 4);
        memcpy(out.data(), data, out.size() * 4);
    } else {
        return n3_fail(RN_ERR_ARGUMENT, "tensor %d holds kind %d, not floating point values", index, r.kind);
    }
    return RN_OK;
}

// a float tensor of exactly `count` values (count < 0: any) to the device
int device_floats(rn_n3_model* m, const rn_archive* a, int index, float** out, long count,
                  std::vector<float>* keep = nullptr) {
    std::vector<float> v;
    N3_CALL(host_floats(a, index, v));
    if (count >= 0 && (long)v.size() != count)
        return n3_fail(RN_ERR_ARGUMENT, "tensor %d holds %zu values, %ld expected", index, v.size(), count);
    if (keep) *keep = v;
    return upload_floats(m, v, out);
}

int matrix(rn_n3_model* m, const rn_archive* a, int index, rn_matrix** out) {
    N3_CALL(rn_matrix_from_archive(a, index, out));
    m->matrices.push_back(*out);
    return RN_OK;
}

// rows of a matrix dequantised on the device, gathered on the host
int dense_rows(const rn_matrix* mat, const std::vector<int>& rows, std::vector<float>& out) {
    out.resize(rows.size() * (size_t)mat->columns);
    for (size_t i = 0; i < rows.size(); ++i)
        N3_CALL(rn_matrix_dequantise_row(mat, rows[i], out.data() + i * mat->columns));
    return RN_OK;
}

// The four projections of a layer that share bits and group as one matrix:
// their packed rows in order, then their norms in order (the same row
// arithmetic; one launch instead of four, QuantisedMatrix::multiply_fused).
int stack_projections(rn_n3_model* m, const rn_archive* a, const int idx[4], N3Layer& y) {
    const rn_matrix* mats[4] = {y.q, y.k, y.v, y.gate};
    for (const rn_matrix* x : mats)
        if (x->bits != y.q->bits || x->group != y.q->group) return RN_OK;
    std::vector<uint8_t> packed, norms;
    int rows = 0;
    for (int i = 0; i < 4; ++i) {
        const uint8_t* data = nullptr;
        size_t n = 0;
        N3_CALL(rn_archive_tensor_bytes(a, idx[i], &data, &n));
        const size_t pb = (size_t)mats[i]->rows * mats[i]->cb.row_bytes;
        const size_t nb = (size_t)mats[i]->rows * (mats[i]->cb.padded / mats[i]->group) * 2;
        packed.insert(packed.end(), data, data + pb);
        norms.insert(norms.end(), data + pb, data + pb + nb);
        rows += mats[i]->rows;
    }
    packed.insert(packed.end(), norms.begin(), norms.end());
    const float* codebook = nullptr;
    int count = 0;
    N3_CALL(rn_archive_codebook(a, &codebook, &count));
    N3_CALL(rn_matrix_create_codebook(packed.data(), packed.size(), rows, y.q->columns, y.q->group, y.q->bits, codebook,
                                      count, &y.qkvg));
    m->matrices.push_back(y.qkvg);
    return RN_OK;
}

// config.rs:61: tables over the orders
int heads_per_order(const rn_geometry& g) { return (int)g.engram_tables / (g.engram_order_count > 1 ? (int)g.engram_order_count : 1); }

bool integer_path(const rn_matrix* x) { return x->bits == 2 || x->bits == 4 || x->bits == 5; }

// phi_stack (device to device copies at open)
int stack_routing_rows(rn_n3_model* m) {
    const int L = (int)m->g.mhc_lanes, layers = (int)m->g.num_layers;
    const size_t rb = m->phi_pre->cb.row_bytes, per = (size_t)(2 * L + L * L) * rb;
    void* q = nullptr;
    N3_CALL(arena_take(m->allocations, m->arena, per * layers, kN3ModelChunk, &q));
    m->phi_stack = static_cast<uint8_t*>(q);
    for (int l = 0; l < layers; ++l) {
        uint8_t* dst = m->phi_stack + per * l;
        N3_HIP(hipMemcpy(dst, m->phi_pre->cb.packed + (size_t)l * L * rb, L * rb, hipMemcpyDeviceToDevice));
        N3_HIP(hipMemcpy(dst + L * rb, m->phi_post->cb.packed + (size_t)l * L * rb, L * rb, hipMemcpyDeviceToDevice));
        N3_HIP(hipMemcpy(dst + 2 * L * rb, m->phi_res->cb.packed + (size_t)l * L * L * rb, (size_t)L * L * rb,
                         hipMemcpyDeviceToDevice));
    }
    return RN_OK;
}

// 16-byte loads a thread of n3_out_kernel for rows of `row_bytes` (64 rows,
// 1024 threads), rounded up to a power of two
int n3_out_loads(int row_bytes) {
    const int need = (64 * (row_bytes / 16) + 1023) / 1024;
    int l = 1;
    while (l < need) l *= 2;
    return l;
}

// The layer boundary kernel (tail, routing, block input) applies: integer-path
// routing matrices whose rows start where the reference takes the panel form
// (2-bit rows on panels of four), at most four lanes, vectors that fit its LDS
// staging, and a stacked q/k/v/gate matrix whose prepared input fits it. The
// batched feed needs this much; its products take either path.
bool boundary_applies(const rn_n3_model* m) {
    const rn_geometry& g = m->g;
    const int L = (int)g.mhc_lanes;
    if (2 * L + L * L > kN3RouteRows || g.d_model > (uint32_t)kN3Hadamard) return false;
    if (g.qkv_conv_taps > (uint32_t)kN3MaxTaps) return false;
    if (m->phi_pre->cb.row_bytes > kN3RouteRowBytes || m->phi_pre->cb.padded / m->phi_pre->group > 64) return false;
    // the input codes four lanes a run: groups of at most 256
    if (m->phi_pre->group > 256) return false;
    if ((2 * L + L * L) * (m->phi_pre->cb.padded / m->phi_pre->group) > kN3Block) return false;
    // the layer boundary stages three vectors and the stream in 1 KB chunks,
    // two a wave (d a multiple of 256), and copies the factors, cond_v and the
    // routing rows in 16-byte units; its norms take squares four a read
    const int d = (int)g.d_model;
    if (d % 256 != 0 || (3 * d + L * d) / 256 > 2 * (kN3Block / 64)) return false;
    if (g.engram_conv_taps > (uint32_t)kN3MaxTaps) return false;  // the boundary's site convolution
    if (m->embedding->cb.padded > kN3Hadamard || m->embedding->group > 256) return false;  // the logits' input
    if (m->phi_pre->cb.row_bytes % 16 != 0) return false;
    auto aligned = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
    const rn_matrix* phis[3] = {m->phi_pre, m->phi_post, m->phi_res};
    for (const rn_matrix* x : phis) {
        if (!integer_path(x) || x->cb.padded > kN3MaxWidth || x->group != m->phi_pre->group ||
            x->cb.padded != m->phi_pre->cb.padded || x->bits != m->phi_pre->bits)
            return false;
        if (x->bits == 2 && L % 4 != 0) return false;
    }
    for (const rn_matrix* x : phis)
        if (!aligned(x->cb.packed)) return false;
    for (const N3Layer& y : m->layers) {
        if (y.qkvg == nullptr) return false;
        for (int f = 0; f < 6; ++f)
            if (!aligned(y.factors[f])) return false;
        if (y.rank == 8 && !aligned(y.cond_v)) return false;
        if (y.qkvg->group > 256 || y.qkvg->cb.padded > kN3Hadamard) return false;
    }
    return true;
}

// The three-kernel step of a push needs, beyond the boundary kernel, the
// attention and output kernels' formats: integer-path projections whose rows
// fit their LDS tiles.
bool fused_applies(const rn_n3_model* m) {
    if (!boundary_applies(m)) return false;
    auto aligned = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
    for (const N3Layer& y : m->layers) {
        if (!aligned(y.out->cb.packed) || !aligned(y.out->cb.norms) || !aligned(y.qkvg->cb.packed)) return false;
        if (y.out->group > 256) return false;
        if (!integer_path(y.qkvg) || y.qkvg->cb.row_bytes > kN3HeadRowBytes) return false;
        if (!integer_path(y.out) || y.out->cb.padded > kN3MaxWidth || y.out->cb.row_bytes > kN3OutRowBytes ||
            y.out->cb.padded / y.out->group > 64 || y.out->cb.row_bytes % 16 != 0)
            return false;
    }
    return true;
}

// ladder.rs:1-29, through the public entry point
int ladder(int layers, int depth, std::vector<int>& active) {
    std::vector<int32_t> chosen((size_t)std::max(layers, 1));
    N3_CALL(rn_ladder_select(layers, depth, chosen.data()));
    active.assign(chosen.begin(), chosen.begin() + depth);
    return RN_OK;
}

}  // namespace

int rn_n3_model_free(rn_n3_model* m) {
    if (!m) return RN_OK;
    for (rn_matrix* x : m->matrices) rn_matrix_free(x);
    for (void* p : m->allocations) (void)hipFree(p);
    delete m;
    return RN_OK;
}

int rn_n3_model_open(const rn_archive* archive, int depth, rn_n3_model** out) {
    N3_REQUIRE(archive && out, "null argument");
    *out = nullptr;
    rn_n3_model* m = new (std::nothrow) rn_n3_model();
    if (!m) return n3_fail(RN_ERR_MEMORY, "out of host memory");
    int rc = [&]() -> int {
        rn_geometry& g = m->g;
        N3_CALL(rn_archive_geometry(archive, &g));
        N3_REQUIRE(g.qk_head_dim == 64 && g.v_head_dim == 64, "head dimensions must be 64 (got %u / %u)", g.qk_head_dim,
                   g.v_head_dim);
        N3_REQUIRE(g.num_kv_heads > 0 && g.num_heads % g.num_kv_heads == 0, "heads must be a multiple of kv heads");
        N3_REQUIRE(g.hada_n == (uint32_t)kN3Hadamard, "the Hadamard size must be 1024 (32 x 32 factors; got %u)",
                   g.hada_n);
        N3_REQUIRE(g.d_model % 8 == 0 && g.d_model <= (uint32_t)kN3Hadamard, "d_model must be a multiple of 8, <= 1024");
        N3_REQUIRE(g.mhc_lanes >= 1 && g.mhc_lanes * g.d_model <= (uint32_t)kN3MaxWidth, "lanes x d_model above %d",
                   kN3MaxWidth);
        N3_REQUIRE(g.num_heads * 64 <= (uint32_t)kN3MaxWidth, "too many heads");
        N3_REQUIRE(g.engram_order_count * (g.engram_order_count ? g.engram_tables / g.engram_order_count : 0) <=
                       (uint32_t)kN3MaxTables,
                   "more than %d engram tables", kN3MaxTables);
        m->output_vocab = g.out_vocab ? (int)g.out_vocab : (int)g.vocab;
        Walk w{archive};
        w.end = (int)g.tensor_count - 1;
        N3_REQUIRE(g.tensor_count >= 1 && w.kind((int)g.tensor_count - 1) == RN_KIND_RAW, "no trailing tokenizer blob");
        N3_CALL(matrix(m, archive, w.take(), &m->embedding));
        const int L = (int)g.num_layers, d = (int)g.d_model;
        N3_REQUIRE(m->embedding->rows >= (int)g.vocab && m->embedding->rows >= m->output_vocab &&
                       m->embedding->columns == d,
                   "embedding [%d][%d] does not cover the vocabulary x d_model", m->embedding->rows,
                   m->embedding->columns);
        m->layers.resize((size_t)L);
        std::vector<float> scalar;
        for (int l = 0; l < L; ++l) {
            N3Layer& y = m->layers[(size_t)l];
            N3_CALL(device_floats(m, archive, w.take(), &y.norm_in, d));
            int proj[4];
            proj[0] = w.take();
            N3_CALL(matrix(m, archive, proj[0], &y.q));
            proj[1] = w.take();
            N3_CALL(matrix(m, archive, proj[1], &y.k));
            proj[2] = w.take();
            N3_CALL(matrix(m, archive, proj[2], &y.v));
            if (g.qkv_conv_taps > 0)
                for (int t = 0; t < 3; ++t)
                    N3_CALL(device_floats(m, archive, w.take(), &y.taps[t],
                                          (long)g.qkv_conv_taps * (t == 0 ? g.num_heads : g.num_kv_heads) * 64));
            N3_CALL(device_floats(m, archive, w.take(), &y.q_norm, 64));
            N3_CALL(device_floats(m, archive, w.take(), &y.k_norm, 64));
            proj[3] = w.take();
            N3_CALL(matrix(m, archive, proj[3], &y.gate));
            N3_CALL(matrix(m, archive, w.take(), &y.out));
            N3_CALL(device_floats(m, archive, w.take(), &y.post_norm, d));
            N3_CALL(host_floats(archive, w.take(), scalar));
            N3_REQUIRE(!scalar.empty(), "attention gate of layer %d is empty", l);
            y.gate_sigmoid = 1.0f / (1.0f + expf(-scalar[0]));  // ops.rs:68-71 with the host's expf
            N3_CALL(device_floats(m, archive, w.take(), &y.pre_norm, d));
            float** diag[5] = {&y.d1, &y.d2, &y.b2, &y.d3, &y.d4};
            for (int i = 0; i < 5; ++i) N3_CALL(device_floats(m, archive, w.take(), diag[i], kN3Hadamard));
            // the six factors and cond_v in one allocation, [w1a .. w3b | cond_v]:
            // the layer boundary stages them as one range
            std::vector<float> tail;
            for (int f = 0; f < 6; ++f) {
                std::vector<float> v;
                const int idx = w.take();
                N3_CALL(host_floats(archive, idx, v));
                N3_REQUIRE(v.size() == 1024, "Hadamard factors must be 32 x 32 (layer %d factor %d)", l, f);
                tail.insert(tail.end(), v.begin(), v.end());
            }
            std::vector<float> cu;
            std::vector<float> cv;
            N3_CALL(host_floats(archive, w.take(), cv));
            tail.insert(tail.end(), cv.begin(), cv.end());
            float* tail_dev = nullptr;
            N3_CALL(upload_floats(m, tail, &tail_dev));
            for (int f = 0; f < 6; ++f) y.factors[f] = tail_dev + (size_t)f * kN3Hadamard;
            y.cond_v = tail_dev + (size_t)6 * kN3Hadamard;
            N3_CALL(device_floats(m, archive, w.take(), &y.cond_u, -1, &cu));
            y.rank = (int)(cu.size() / kN3Hadamard);  // hadamard.rs:39
            N3_REQUIRE(y.rank >= 1 && y.rank <= 64 && cu.size() == (size_t)y.rank * kN3Hadamard &&
                           cv.size() == (size_t)y.rank * d,
                       "condition tensors of layer %d: rank %d (1..64), cond_v [d_model][rank]", l, y.rank);
            const bool same = y.q->columns == d && y.k->columns == d && y.v->columns == d && y.gate->columns == d;
            N3_REQUIRE(same, "projections of layer %d must take d_model columns", l);
            N3_REQUIRE(y.q->rows == (int)(g.num_heads * 64) && y.k->rows == (int)(g.num_kv_heads * 64) &&
                           y.v->rows == (int)(g.num_kv_heads * 64) && y.gate->rows == (int)(g.num_heads * 64) &&
                           y.out->rows == d,
                       "projection shapes of layer %d do not match the geometry", l);
            N3_REQUIRE(y.q->cb.padded == y.k->cb.padded && y.q->cb.padded == y.v->cb.padded &&
                           y.q->cb.padded == y.gate->cb.padded,
                       "projections of layer %d must share their padded width", l);
            N3_CALL(stack_projections(m, archive, proj, y));
        }
        N3_CALL(device_floats(m, archive, w.take(), &m->a_pre, L, &m->a_pre_h));
        N3_CALL(device_floats(m, archive, w.take(), &m->a_post, L, &m->a_post_h));
        N3_CALL(device_floats(m, archive, w.take(), &m->a_res, L, &m->a_res_h));
        N3_CALL(device_floats(m, archive, w.take(), &m->b_pre, (long)L * g.mhc_lanes, &m->b_pre_h));
        N3_CALL(device_floats(m, archive, w.take(), &m->b_post, (long)L * g.mhc_lanes, &m->b_post_h));
        N3_CALL(device_floats(m, archive, w.take(), &m->b_res, (long)L * g.mhc_lanes * g.mhc_lanes, &m->b_res_h));
        N3_CALL(matrix(m, archive, w.take(), &m->phi_pre));
        N3_CALL(matrix(m, archive, w.take(), &m->phi_post));
        N3_CALL(matrix(m, archive, w.take(), &m->phi_res));
        const int lanes = (int)g.mhc_lanes;
        N3_REQUIRE(m->phi_pre->rows == L * lanes && m->phi_post->rows == L * lanes &&
                       m->phi_res->rows == L * lanes * lanes && m->phi_pre->columns == lanes * d &&
                       m->phi_post->columns == lanes * d && m->phi_res->columns == lanes * d,
                   "routing matrices do not match layers x lanes over the lane stream");
        for (int p = 0; p < 2; ++p) {  // hadamard.rs:36: floats, `as usize`
            std::vector<float> v;
            N3_CALL(host_floats(archive, w.take(), v));
            N3_REQUIRE(v.size() == (size_t)kN3Hadamard, "permutation %d has %zu entries", p, v.size());
            std::vector<int32_t> perm(v.size());
            for (size_t i = 0; i < v.size(); ++i) {
                perm[i] = (int32_t)v[i];
                N3_REQUIRE(perm[i] >= 0 && perm[i] < kN3Hadamard, "permutation %d entry out of range", p);
            }
            void* dp = nullptr;
            N3_CALL(arena_take(m->allocations, m->arena, perm.size() * 4, kN3ModelChunk, &dp));
            N3_HIP(hipMemcpy(dp, perm.data(), perm.size() * 4, hipMemcpyHostToDevice));
            m->perm[p] = (int32_t*)dp;
        }
        m->engrams.resize(g.engram_site_count);
        for (N3Engram& e : m->engrams) {
            N3_CALL(matrix(m, archive, w.take(), &e.tables));
            N3_CALL(matrix(m, archive, w.take(), &e.key));
            N3_CALL(matrix(m, archive, w.take(), &e.value));
            N3_CALL(device_floats(m, archive, w.take(), &e.taps, (long)g.engram_conv_taps * d));
            N3_REQUIRE(e.key->rows == d && e.value->rows == d, "engram projections must give d_model rows");
            N3_REQUIRE(e.key->cb.padded == e.value->cb.padded, "engram projections must share their width");
            N3_REQUIRE(e.tables->columns == (int)g.engram_sub_dim && e.tables->cb.padded == e.tables->columns,
                       "engram tables must hold sub_dim columns, a whole number of groups");
            const int tables = (int)g.engram_order_count * heads_per_order(g);
            N3_REQUIRE(e.key->columns == tables * (int)g.engram_sub_dim && tables * (int)g.engram_sub_dim <= kN3MaxWidth &&
                           e.tables->rows >= tables * (int)g.engram_slots && g.engram_slots > 0,
                       "engram projections must take tables x sub_dim columns (at most %d)", kN3MaxWidth);
        }
        N3_CALL(device_floats(m, archive, w.take(), &m->final_norm, d));
        if (w.failed) return n3_fail(RN_ERR_ARGUMENT, "directory ends before the canonical tensor list");
        if (depth <= 0) depth = L;
        N3_CALL(ladder(L, depth, m->active));
        N3_REQUIRE(!m->active.empty(), "depth %d selects no layers", depth);
        // probe heads (layout.rs:228-246; heads.rs:33-82 with with_rows)
        if (w.next < w.end && w.kind(w.next) == RN_KIND_HALF) {
            std::vector<float> codes;
            N3_CALL(host_floats(archive, w.take(), codes));
            for (float cf : codes) {
                const int code = (int)lroundf(cf);
                N3_REQUIRE(code >= 1 && code <= 3, "unrecognised head manifest code");
                N3Head h;
                h.code = code;
                rn_matrix *probes = nullptr, *query = nullptr;
                N3_CALL(matrix(m, archive, w.take(), &probes));
                std::vector<float> gain, row_bias;
                N3_CALL(host_floats(archive, w.take(), gain));
                N3_CALL(matrix(m, archive, w.take(), &query));
                N3_CALL(host_floats(archive, w.take(), row_bias));
                N3_CALL(matrix(m, archive, w.take(), &h.projection));
                N3_CALL(device_floats(m, archive, w.take(), &h.bias, h.projection->rows));
                if (code == 3) w.take();  // calibration
                const int rows_all = L + 1, k = probes->rows / rows_all;
                h.width = probes->columns;
                h.per_layer = k;
                h.queries = query->rows;
                h.layers = (int)m->active.size() + 1;
                N3_REQUIRE(h.width == d && k >= 1 && probes->rows == rows_all * k, "probe head rows must be layers x k over d_model");
                N3_REQUIRE(query->columns == d && h.projection->columns == h.queries * d &&
                               gain.size() == (size_t)rows_all * k && row_bias.size() == (size_t)h.queries * rows_all * k,
                           "probe head tensors do not match its probes and queries");
                N3_REQUIRE(h.queries * d <= kN3MaxWidth * 16, "too many probe queries");
                N3_REQUIRE(h.layers * k <= 1024, "more than 1024 probe slots");
                std::vector<int> rows, qrows;
                std::vector<float> sel_gain, sel_bias;
                const int old_slots = rows_all * k;
                for (int ri = 0; ri < h.layers; ++ri) {
                    const int row = ri == 0 ? 0 : m->active[(size_t)ri - 1] + 1;
                    for (int p = 0; p < k; ++p) {
                        rows.push_back(row * k + p);
                        sel_gain.push_back(gain[(size_t)row * k + p]);
                    }
                }
                for (int q = 0; q < h.queries; ++q) {
                    qrows.push_back(q);
                    for (int ri = 0; ri < h.layers; ++ri) {
                        const int row = ri == 0 ? 0 : m->active[(size_t)ri - 1] + 1;
                        for (int p = 0; p < k; ++p) sel_bias.push_back(row_bias[(size_t)q * old_slots + row * k + p]);
                    }
                }
                std::vector<float> dense;
                N3_CALL(dense_rows(probes, rows, dense));
                N3_CALL(upload_floats(m, dense, &h.probes));
                N3_CALL(dense_rows(query, qrows, dense));
                N3_CALL(upload_floats(m, dense, &h.query));
                N3_CALL(upload_floats(m, sel_gain, &h.gain));
                N3_CALL(upload_floats(m, sel_bias, &h.row_bias));
                m->heads.push_back(h);
            }
        }
        if (w.failed) return n3_fail(RN_ERR_ARGUMENT, "directory ends inside the probe heads");
        m->fused = fused_applies(m);
        // the boundary kernel (pushes of the fused step and every batched feed)
        // reads the routing rows from this stack
        if (boundary_applies(m)) N3_CALL(stack_routing_rows(m));
        N3_REQUIRE(w.next == w.end, "%d tensors follow the heads (an audio encoder is not part of this model)",
                   w.end - w.next);
        return RN_OK;
    }();
    if (rc != RN_OK) {
        rn_n3_model_free(m);
        return rc;
    }
    *out = m;
    return RN_OK;
}

int rn_n3_model_active_layers(const rn_n3_model* m, int* layers, int* count) {
    N3_REQUIRE(m && count, "null argument");
    *count = (int)m->active.size();
    if (layers) std::copy(m->active.begin(), m->active.end(), layers);
    return RN_OK;
}

int rn_n3_model_output_vocab(const rn_n3_model* m, int* count) {
    N3_REQUIRE(m && count, "null argument");
    *count = m->output_vocab;
    return RN_OK;
}

struct N3CacheDev {
    int8_t *keys = nullptr, *values = nullptr;
    float *key_scales = nullptr, *value_scales = nullptr, *hist = nullptr;
};

struct rn_n3_session {
    const rn_n3_model* m = nullptr;
    int capacity = 0, length = 0;
    bool fused = false;  // three kernels a layer; RN_N3_PATH=stepwise forces one launch per piece
    hipStream_t stream = nullptr;
    rn_lanes* lanes = nullptr;
    std::vector<N3CacheDev> caches;
    std::vector<float*> rings, ekey, evalue, site_rot, site_raw;  // per engram site
    std::vector<void*> allocations;  // every device buffer of the session lives in these chunks
    std::vector<size_t> allocation_bytes;
    N3Arena arena;
    float *stream_a = nullptr, *stream_b = nullptr, *input = nullptr, *post = nullptr, *residual = nullptr;
    float *x = nullptr, *rotated = nullptr, *prod = nullptr, *attended = nullptr;
    void* codes = nullptr;         // the projections' input codes (int4 a run of 16)
    float* code_scales = nullptr;
    float* lrot = nullptr;     // the logits' input prepared by the last fused push (lrot_ready)
    bool lrot_ready = false;
    uint32_t* tokens_dev = nullptr;  // the tokens pushed so far [capacity]
    uint32_t* next_dev = nullptr;    // the greedy argmax of the last logits
    uint32_t* ids_dev = nullptr;     // greedy ids [capacity]
    uint8_t* allowed_dev = nullptr;  // the grammar's mask [output_vocab] (rn_n3_session_choose_allowed)
    Choice* choice_dev = nullptr;
    uint32_t* turn_host = nullptr;   // pinned: the last two greedy tokens of a turn (rn_n3_session_run_turn)
    hipEvent_t turn_done[2] = {nullptr, nullptr};
    float *attn_out = nullptr, *gathered = nullptr, *eraw = nullptr, *qscales = nullptr;
    int8_t* qcodes = nullptr;
    float *cells = nullptr, *hidden = nullptr, *logits = nullptr, *cos = nullptr, *sin = nullptr;
    std::vector<float*> peak, total, weighted;
    float *readouts = nullptr, *pooled = nullptr, *head_out = nullptr;
    // a batched feed's vectors, kN3FeedChunk tokens of each (taken on the first feed)
    struct Run {
        bool ready = false;
        float *stream_a = nullptr, *stream_b = nullptr, *attn = nullptr, *x = nullptr, *input = nullptr;
        float *post = nullptr, *residual = nullptr, *rotated = nullptr, *prod = nullptr, *attended = nullptr;
        float *qscales = nullptr, *cells = nullptr, *gathered = nullptr, *eraw = nullptr;
        int8_t* qcodes = nullptr;
        std::vector<float*> ekey, evalue;
    } run;
};

namespace {

int alloc(rn_n3_session* s, size_t bytes, void** out) {
    void* p = nullptr;
    N3_CALL(arena_take(s->allocations, s->arena, bytes, kN3SessionChunk, &p, &s->allocation_bytes));
    N3_HIP(hipMemsetAsync(p, 0, std::max<size_t>(bytes, 256), s->stream));
    *out = p;
    return RN_OK;
}
template <typename T>
int alloc_n(rn_n3_session* s, size_t n, T** out) {
    void* p = nullptr;
    N3_CALL(alloc(s, n * sizeof(T), &p));
    *out = (T*)p;
    return RN_OK;
}

// QuantisedMatrix::multiply_vector on a rotated input (matrix.rs:155-165): the
// integer path for 2-, 4-bit and ternary matrices, the float path otherwise
int product(const rn_matrix* mat, const float* rotated, float* y, hipStream_t st) {
    if (mat->bits == 1 || mat->bits == 3)
        N3_HIP(launch_codebook_float(mat->cb, rotated, 1, y, false, st));
    else
        N3_HIP(launch_codebook_product(mat->cb, rotated, 1, y, nullptr, st));
    return RN_OK;
}

// QuantisedMatrix::multiply_batch (matrix.rs:330-389) of count rotated inputs:
// the integer path per token, the float path's batch tile otherwise
int product_run(const rn_matrix* mat, const float* rotated, int count, float* y, hipStream_t st) {
    if (mat->bits == 1 || mat->bits == 3)
        N3_HIP(launch_codebook_float(mat->cb, rotated, count, y, true, st));
    else
        N3_HIP(launch_codebook_product(mat->cb, rotated, count, y, nullptr, st));
    return RN_OK;
}

int rotate(const rn_matrix* mat, const float* x, float* rotated, hipStream_t st) {
    N3_HIP(launch_codebook_rotate(x, 1, mat->columns, mat->cb.padded, mat->group, mat->cb.wht_scale, rotated, st));
    return RN_OK;
}

// attention.rs:172-178: the window's first position unless the layer is global
int window_first(const rn_geometry& g, int layer, int total) {
    if (g.sliding_window > 0 && !((g.global_layers >> layer) & 1))
        return total > (int)g.sliding_window ? total - (int)g.sliding_window : 0;
    return 0;
}

// the positions a layer's query sees (0: all of them)
int layer_window(const rn_geometry& g, int layer) {
    return g.sliding_window > 0 && !((g.global_layers >> layer) & 1) ? (int)g.sliding_window : 0;
}

int site_of(const rn_n3_model* m, int layer) {  // config.rs:89-91
    for (uint32_t e = 0; e < m->g.engram_site_count; ++e)
        if ((int)m->g.engram_sites[e] == layer) return (int)e;
    return -1;
}

bool site_active(const rn_n3_model* m, int site) {
    return std::find(m->active.begin(), m->active.end(), (int)m->g.engram_sites[site]) != m->active.end();
}



}  // namespace

int rn_n3_session_free(rn_n3_session* s) {
    if (!s) return RN_OK;
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    if (s->lanes) rn_lanes_free(s->lanes);
    for (void* p : s->allocations) (void)hipFree(p);
    for (hipEvent_t e : s->turn_done)
        if (e) (void)hipEventDestroy(e);
    if (s->turn_host) (void)hipHostFree(s->turn_host);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    delete s;
    return RN_OK;
}

int rn_n3_session_create(const rn_n3_model* m, int capacity, rn_n3_session** out) {
    N3_REQUIRE(m && out, "null argument");
    N3_REQUIRE(capacity >= 1 && capacity <= kN3MaxAttend, "capacity must be 1..%d (got %d)", kN3MaxAttend, capacity);
    *out = nullptr;
    rn_n3_session* s = new (std::nothrow) rn_n3_session();
    if (!s) return n3_fail(RN_ERR_MEMORY, "out of host memory");
    s->m = m;
    s->capacity = capacity;
    {
        const char* path = getenv("RN_N3_PATH");
        s->fused = m->fused && !(path && strcmp(path, "stepwise") == 0);
    }
    int rc = [&]() -> int {
        const rn_geometry& g = m->g;
        const int d = (int)g.d_model, L = (int)g.num_layers, lanes = (int)g.mhc_lanes, H = (int)g.num_heads,
                  KV = (int)g.num_kv_heads;
        N3_HIP(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
        N3_CALL(rn_lanes_create(lanes, d, L, m->a_pre_h.data(), m->a_post_h.data(), m->a_res_h.data(),
                                m->b_pre_h.data(), m->b_post_h.data(), m->b_res_h.data(), m->phi_pre, m->phi_post,
                                m->phi_res, &s->lanes));
        s->caches.resize((size_t)L);
        const int qkv = (H + 2 * KV) * 64, taps = std::max(1, (int)g.qkv_conv_taps);
        for (N3CacheDev& c : s->caches) {
            N3_CALL(alloc_n(s, (size_t)KV * capacity * 64, &c.keys));
            N3_CALL(alloc_n(s, (size_t)KV * capacity * 64, &c.values));
            N3_CALL(alloc_n(s, (size_t)KV * capacity, &c.key_scales));
            N3_CALL(alloc_n(s, (size_t)KV * capacity, &c.value_scales));
            N3_CALL(alloc_n(s, (size_t)taps * qkv, &c.hist));
        }
        const int keep = std::max(1, ((int)g.engram_conv_taps - 1) * (int)g.engram_conv_dilation + 1);
        s->rings.resize(g.engram_site_count);
        s->ekey.resize(g.engram_site_count);
        s->evalue.resize(g.engram_site_count);
        s->site_rot.resize(g.engram_site_count);
        s->site_raw.resize(g.engram_site_count);
        for (uint32_t e = 0; e < g.engram_site_count; ++e) {
            N3_CALL(alloc_n(s, (size_t)keep * d, &s->rings[e]));
            N3_CALL(alloc_n(s, (size_t)d, &s->ekey[e]));
            N3_CALL(alloc_n(s, (size_t)d, &s->evalue[e]));
            N3_CALL(alloc_n(s, (size_t)m->engrams[e].key->cb.padded, &s->site_rot[e]));
            N3_CALL(alloc_n(s, (size_t)d, &s->site_raw[e]));
        }
        int widest = std::max(lanes * d, qkv + H * 64);
        for (const N3Engram& e : m->engrams) widest = std::max(widest, e.key->cb.padded);
        for (const N3Head& h : m->heads) widest = std::max(widest, h.projection->cb.padded);
        widest = std::max(widest, m->embedding->cb.padded);
        N3_CALL(alloc_n(s, (size_t)lanes * d, &s->stream_a));
        N3_CALL(alloc_n(s, (size_t)lanes * d, &s->stream_b));
        N3_CALL(alloc_n(s, 64, &s->post));
        N3_CALL(alloc_n(s, 256, &s->residual));
        N3_CALL(alloc_n(s, (size_t)widest, &s->rotated));
        N3_CALL(alloc_n(s, (size_t)m->embedding->cb.padded, &s->lrot));
        N3_CALL(alloc_n(s, (size_t)qkv + H * 64, &s->prod));
        N3_CALL(alloc_n(s, (size_t)H * 64, &s->attended));
        N3_CALL(alloc(s, (size_t)kN3Hadamard, &s->codes));
        N3_CALL(alloc_n(s, (size_t)capacity, &s->tokens_dev));
        N3_CALL(alloc_n(s, 64, &s->next_dev));
        N3_CALL(alloc_n(s, (size_t)capacity, &s->ids_dev));
        N3_CALL(alloc_n(s, (size_t)m->output_vocab, &s->allowed_dev));
        N3_CALL(alloc_n(s, 1, &s->choice_dev));
        N3_CALL(alloc_n(s, 64, &s->code_scales));
        // the output projection, x and the routed input one after another: the
        // layer boundary stages them as one range
        N3_CALL(alloc_n(s, (size_t)3 * d, &s->attn_out));
        s->x = s->attn_out + d;
        s->input = s->attn_out + 2 * (size_t)d;
        N3_CALL(alloc_n(s, (size_t)kN3MaxWidth, &s->gathered));
        N3_CALL(alloc_n(s, (size_t)d, &s->eraw));
        N3_CALL(alloc_n(s, (size_t)H, &s->qscales));
        N3_CALL(alloc_n(s, (size_t)H * 64, &s->qcodes));
        N3_CALL(alloc_n(s, (size_t)(m->active.size() + 1) * d, &s->cells));
        N3_CALL(alloc_n(s, (size_t)d, &s->hidden));
        N3_CALL(alloc_n(s, (size_t)m->output_vocab, &s->logits));
        // the rotary table (ops.rs:127-141): angle = position as f32 * frequency
        std::vector<float> cs((size_t)capacity * 32), sn((size_t)capacity * 32);
        for (int p = 0; p < capacity; ++p)
            for (int i = 0; i < 32; ++i) {
                const float freq = 1.0f / powf(g.rope_theta, (2.0f * (float)i) / 64.0f);
                const float angle = (float)p * freq;
                cs[(size_t)p * 32 + i] = cosf(angle);
                sn[(size_t)p * 32 + i] = sinf(angle);
            }
        N3_CALL(alloc_n(s, cs.size(), &s->cos));
        N3_CALL(alloc_n(s, sn.size(), &s->sin));
        N3_HIP(hipMemcpyAsync(s->cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, s->stream));
        N3_HIP(hipMemcpyAsync(s->sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice, s->stream));
        size_t readouts = 0, pooled = 0, outs = 0;
        for (const N3Head& h : m->heads) {
            const int slots = h.layers * h.per_layer;
            float *pk = nullptr, *tt = nullptr, *wt = nullptr;
            N3_CALL(alloc_n(s, (size_t)slots, &pk));
            N3_CALL(alloc_n(s, (size_t)slots, &tt));
            N3_CALL(alloc_n(s, (size_t)slots * h.width, &wt));
            std::vector<float> ninf((size_t)slots, -INFINITY);
            N3_HIP(hipMemcpyAsync(pk, ninf.data(), ninf.size() * 4, hipMemcpyHostToDevice, s->stream));
            s->peak.push_back(pk);
            s->total.push_back(tt);
            s->weighted.push_back(wt);
            readouts = std::max(readouts, (size_t)slots * h.width);
            pooled = std::max(pooled, (size_t)h.queries * h.width);
            outs = std::max(outs, (size_t)h.projection->rows);
        }
        N3_CALL(alloc_n(s, std::max<size_t>(readouts, 1), &s->readouts));
        N3_CALL(alloc_n(s, std::max<size_t>(pooled, 1), &s->pooled));
        N3_CALL(alloc_n(s, std::max<size_t>(outs, 1), &s->head_out));
        N3_HIP(hipStreamSynchronize(s->stream));
        return RN_OK;
    }();
    if (rc != RN_OK) {
        rn_n3_session_free(s);
        return rc;
    }
    *out = s;
    return RN_OK;
}

namespace {

// The layers of one push, one launch per piece (any format); the hidden state
// at the end.
int stepwise_layers(rn_n3_session* s, int position, float* cur, float* nxt) {
    const rn_n3_model* m = s->m;
    const rn_geometry& g = m->g;
    const int d = (int)g.d_model, lanes = (int)g.mhc_lanes, H = (int)g.num_heads, KV = (int)g.num_kv_heads;
    hipStream_t st = s->stream;
    const int qw = H * 64, kw = KV * 64, qkv = qw + 2 * kw;
    for (size_t slot = 0; slot < m->active.size(); ++slot) {
        const int layer = m->active[slot];
        const N3Layer& y = m->layers[(size_t)layer];
        N3CacheDev& c = s->caches[(size_t)layer];
        N3_CALL(rn_lanes_route(s->lanes, layer, (int)slot, cur, s->input, s->post, s->residual, st));
        const int site = site_of(m, layer);
        N3BlockInParams bi{s->input, site >= 0 ? s->ekey[(size_t)site] : nullptr,
                           site >= 0 ? s->evalue[(size_t)site] : nullptr, y.norm_in, d, s->x, y.q->cb.padded,
                           y.q->group, y.q->cb.wht_scale, s->rotated};
        rn_launch(n3_block_in_kernel, dim3(1), dim3(kN3Block), 0, st, bi);
        N3_HIP(hipGetLastError());
        if (y.qkvg != nullptr) {
            N3_CALL(product(y.qkvg, s->rotated, s->prod, st));
        } else {
            N3_CALL(product(y.q, s->rotated, s->prod, st));
            N3_CALL(product(y.k, s->rotated, s->prod + qw, st));
            N3_CALL(product(y.v, s->rotated, s->prod + qw + kw, st));
            N3_CALL(product(y.gate, s->rotated, s->prod + qkv, st));
        }
        N3QkvParams qp{};
        qp.prod = s->prod;
        qp.hist = c.hist;
        for (int t = 0; t < 3; ++t) qp.taps[t] = y.taps[t];
        qp.ntaps = (int)g.qkv_conv_taps;
        qp.position = position;
        qp.H = H;
        qp.KV = KV;
        qp.cap = s->capacity;
        qp.q_norm = y.q_norm;
        qp.k_norm = y.k_norm;
        qp.cos_row = s->cos + (size_t)position * 32;
        qp.sin_row = s->sin + (size_t)position * 32;
        qp.qcodes = s->qcodes;
        qp.qscales = s->qscales;
        qp.keys = c.keys;
        qp.key_scales = c.key_scales;
        qp.values = c.values;
        qp.value_scales = c.value_scales;
        rn_launch(n3_qkv_kernel, dim3(H + 2 * KV), dim3(64), 0, st, qp);
        N3_HIP(hipGetLastError());
        N3AttendParams ap{s->qcodes, s->qscales, c.keys, c.key_scales, c.values, c.value_scales, s->prod + qkv,
                          s->capacity, position, layer_window(g, layer), H / KV, 1.0f / sqrtf(64.0f), s->attended, 0};
        rn_launch(n3_attend_kernel, dim3(H), dim3(256), 0, st, ap);
        N3_HIP(hipGetLastError());
        rn_launch(n3_fake_quantise_kernel, dim3(1), dim3(kN3Block), 0, st, (const float*)s->attended, H * 64,
                  y.out->cb.padded, y.out->group, y.out->cb.wht_scale, s->rotated);
        N3_HIP(hipGetLastError());
        N3_CALL(product(y.out, s->rotated, s->attn_out, st));
        N3BlockOutParams bo{};
        bo.attention = s->attn_out;
        bo.post_norm = y.post_norm;
        bo.gate = y.gate_sigmoid;
        bo.pre_norm = y.pre_norm;
        bo.d1 = y.d1;
        bo.d2 = y.d2;
        bo.b2 = y.b2;
        bo.d3 = y.d3;
        bo.d4 = y.d4;
        for (int f = 0; f < 6; ++f) bo.factors[f] = y.factors[f];
        bo.cond_v = y.cond_v;
        bo.cond_u = y.cond_u;
        bo.rank = y.rank;
        bo.perm1 = m->perm[0];
        bo.perm2 = m->perm[1];
        bo.x = s->x;
        bo.input = s->input;
        bo.post = s->post;
        bo.residual = s->residual;
        bo.stream = cur;
        bo.d = d;
        bo.lanes = lanes;
        bo.next = nxt;
        bo.cell = s->cells + (slot + 1) * (size_t)d;
        rn_launch(n3_block_out_kernel, dim3(1), dim3(kN3Block), 0, st, bo);
        N3_HIP(hipGetLastError());
        std::swap(cur, nxt);
    }
    rn_launch(n3_final_kernel, dim3(1), dim3(kN3Block), 0, st, (const float*)cur, d, lanes,
              (const float*)m->final_norm, s->hidden);
    N3_HIP(hipGetLastError());
    return RN_OK;
}

// The layers of one push in three kernels a layer (n3_attention, n3_out,
// n3_boundary); the routing of the first layer by a boundary without a tail.
int fused_layers(rn_n3_session* s, int position, float* cur, float* nxt) {
    const rn_n3_model* m = s->m;
    const rn_geometry& g = m->g;
    const int d = (int)g.d_model, lanes = (int)g.mhc_lanes, H = (int)g.num_heads, KV = (int)g.num_kv_heads;
    hipStream_t st = s->stream;
    const size_t layers = m->active.size();
    auto route_into = [&](N3BoundaryParams& b, size_t slot) {
        const int layer = m->active[slot];
        const N3Layer& y = m->layers[(size_t)layer];
        const int site = site_of(m, layer);
        b.route = 1;
        b.layer = layer;
        b.slot = (int)slot;
        b.phi_pre = m->phi_pre->cb;
        b.phi_post = m->phi_post->cb;
        b.phi_res = m->phi_res->cb;
        b.a_pre = m->a_pre;
        b.a_post = m->a_post;
        b.a_res = m->a_res;
        b.b_pre = m->b_pre;
        b.b_post = m->b_post;
        b.b_res = m->b_res;
        b.input = s->input;
        b.post = s->post;
        b.residual = s->residual;
        b.key = site >= 0 ? s->ekey[(size_t)site] : nullptr;
        b.value = site >= 0 ? s->evalue[(size_t)site] : nullptr;
        if (site >= 0) {  // the site's convolution in the boundary (enqueue_sites leaves it)
            b.raw = s->site_raw[(size_t)site];
            b.ring = s->rings[(size_t)site];
            b.taps = m->engrams[(size_t)site].taps;
            b.position = position;
            b.keep = std::max(1, ((int)g.engram_conv_taps - 1) * (int)g.engram_conv_dilation + 1);
            b.ntaps = (int)g.engram_conv_taps;
            b.dilation = (int)g.engram_conv_dilation;
        }
        b.norm_in = y.norm_in;
        b.x = s->x;
        b.qpadded = y.qkvg->cb.padded;
        b.qgroup = y.qkvg->group;
        b.qib = y.qkvg->bits == 5 ? 2 : y.qkvg->bits;
        b.qscale = y.qkvg->cb.wht_scale;
        b.codes = reinterpret_cast<int4*>(s->codes);
        b.code_scales = s->code_scales;
        b.phi_rows = m->phi_stack + (size_t)layer * (2 * lanes + lanes * lanes) * m->phi_pre->cb.row_bytes;
    };
    {
        N3BoundaryParams b{};
        b.stream = cur;
        b.d = d;
        b.lanes = lanes;
        route_into(b, 0);
        rn_launch(n3_boundary_kernel, dim3(1), dim3(kN3Block), 0, st, b);
        N3_HIP(hipGetLastError());
    }
    const int qw = H * 64;
    for (size_t slot = 0; slot < layers; ++slot) {
        const int layer = m->active[slot];
        const N3Layer& y = m->layers[(size_t)layer];
        N3CacheDev& c = s->caches[(size_t)layer];
        const int total = position + 1, first = window_first(g, layer, total);
        N3AttentionParams ap{};
        ap.qkvg = y.qkvg->cb;
        ap.codes = reinterpret_cast<const int4*>(s->codes);
        ap.code_scales = s->code_scales;
        ap.hist = c.hist;
        for (int t = 0; t < 3; ++t) ap.taps[t] = y.taps[t];
        ap.ntaps = (int)g.qkv_conv_taps;
        ap.position = position;
        ap.H = H;
        ap.KV = KV;
        ap.cap = s->capacity;
        ap.first = first;
        ap.count = total - first;
        ap.q_norm = y.q_norm;
        ap.k_norm = y.k_norm;
        ap.cos_row = s->cos + (size_t)position * 32;
        ap.sin_row = s->sin + (size_t)position * 32;
        ap.keys = c.keys;
        ap.key_scales = c.key_scales;
        ap.values = c.values;
        ap.value_scales = c.value_scales;
        ap.out = s->attended;
        rn_launch(n3_attention_kernel, dim3(H), dim3(kN3AttendThreads), 0, st, ap);
        N3_HIP(hipGetLastError());
        N3OutParams op{y.out->cb, s->attended, qw, s->attn_out};
        const dim3 out_grid((unsigned)((y.out->rows + 63) / 64));
        switch (n3_out_loads(y.out->cb.row_bytes)) {
            case 1: rn_launch(n3_out_kernel<1>, out_grid, dim3(1024), 0, st, op); break;
            case 2: rn_launch(n3_out_kernel<2>, out_grid, dim3(1024), 0, st, op); break;
            default: rn_launch(n3_out_kernel<4>, out_grid, dim3(1024), 0, st, op); break;
        }
        N3_HIP(hipGetLastError());
        N3BoundaryParams b{};
        b.tail = 1;
        N3BlockOutParams& bo = b.t;
        bo.attention = s->attn_out;
        bo.post_norm = y.post_norm;
        bo.gate = y.gate_sigmoid;
        bo.pre_norm = y.pre_norm;
        bo.d1 = y.d1;
        bo.d2 = y.d2;
        bo.b2 = y.b2;
        bo.d3 = y.d3;
        bo.d4 = y.d4;
        for (int f = 0; f < 6; ++f) bo.factors[f] = y.factors[f];
        bo.cond_v = y.cond_v;
        bo.cond_u = y.cond_u;
        bo.rank = y.rank;
        bo.perm1 = m->perm[0];
        bo.perm2 = m->perm[1];
        bo.x = s->x;
        bo.input = s->input;
        bo.post = s->post;
        bo.residual = s->residual;
        bo.stream = cur;
        bo.d = d;
        bo.lanes = lanes;
        bo.next = nxt;
        bo.cell = s->cells + (slot + 1) * (size_t)d;
        b.d = d;
        b.lanes = lanes;
        if (slot + 1 < layers) {
            route_into(b, slot + 1);
        } else {
            b.final = 1;
            b.final_norm = m->final_norm;
            b.hidden = s->hidden;
            b.logits_in = s->lrot;
            b.lpadded = m->embedding->cb.padded;
            b.lgroup = m->embedding->group;
            b.lwht = m->embedding->cb.wht_scale;
        }
        rn_launch(n3_boundary_kernel, dim3(1), dim3(kN3Block), 0, st, b);
        N3_HIP(hipGetLastError());
        std::swap(cur, nxt);
    }
    return RN_OK;
}

}  // namespace

namespace {

// The engram sites of a push at `position` (engram.rs:30-112); the value
// convolutions only with `conv`
int enqueue_sites(rn_n3_session* s, int position, bool conv, const N3GatherSites* embed) {
    const rn_n3_model* m = s->m;
    const rn_geometry& g = m->g;
    const int d = (int)g.d_model;
    hipStream_t st = s->stream;
    const int hpo = heads_per_order(g), tables = (int)g.engram_order_count * hpo;
    const int keep = std::max(1, ((int)g.engram_conv_taps - 1) * (int)g.engram_conv_dilation + 1);
    std::vector<int> act;
    for (uint32_t e = 0; e < g.engram_site_count; ++e)
        if (site_active(m, (int)e)) act.push_back((int)e);
    for (size_t b0 = 0; b0 < std::max<size_t>(act.size(), 1); b0 += kN3MaxSites / 2) {  // two products a site
        const int ns = (int)std::min(act.size() - std::min(b0, act.size()), (size_t)kN3MaxSites / 2);
        N3GatherSites gs{};
        if (embed != nullptr && b0 == 0) gs = *embed;  // the first launch also embeds the push's token
        gs.sites = ns;
        N3ConvSites cs{};
        CodebookJobs jobs{};
        bool joint = true;
        for (int k = 0; k < ns; ++k) {
            const int e = act[b0 + (size_t)k];
            const N3Engram& eg = m->engrams[(size_t)e];
            N3GatherParams& gp = gs.site[k];
            gp.tables = eg.tables->cb;
            gp.count = tables;
            gp.sub = (int)g.engram_sub_dim;
            gp.slots = (int)g.engram_slots;
            gp.position = position;
            gp.tokens = s->tokens_dev;
            gp.heads_per_order = hpo;
            gp.stride = g.engram_seed_heads == 0 ? hpo : (int)g.engram_seed_heads;
            for (int o = 0; o < 4; ++o) gp.orders[o] = (int)g.engram_orders[o];
            gp.rotated = s->site_rot[(size_t)e];
            gp.rpadded = eg.key->cb.padded;
            gp.rgroup = eg.key->group;
            gp.rwht = eg.key->cb.wht_scale;
            jobs.job[2 * k] = CodebookJob{eg.key->cb, s->site_rot[(size_t)e], s->ekey[(size_t)e]};
            jobs.job[2 * k + 1] = CodebookJob{eg.value->cb, s->site_rot[(size_t)e], s->site_raw[(size_t)e]};
            joint = joint && integer_path(eg.key) && integer_path(eg.value);
            cs.raw[k] = s->site_raw[(size_t)e];
            cs.ring[k] = s->rings[(size_t)e];
            cs.taps[k] = eg.taps;
            cs.value[k] = s->evalue[(size_t)e];
        }
        rn_launch(n3_gather_kernel, dim3(1, ns + (gs.embed ? 1 : 0)), dim3(kN3Block), 0, st, gs);
        N3_HIP(hipGetLastError());
        if (ns == 0) continue;
        bool same = joint;
        for (int j = 1; j < 2 * ns; ++j) {
            const CodebookParams &a = jobs.job[0].p, &b = jobs.job[j].p;
            same = same && a.bits == b.bits && a.group == b.group && a.padded == b.padded && a.rows == b.rows &&
                   a.cpr == b.cpr;
        }
        if (same && launch_codebook_product_jobs(jobs, 2 * ns, st) == hipSuccess) {
        } else {
            (void)hipGetLastError();
            for (int k = 0; k < ns; ++k) {
                const N3Engram& eg = m->engrams[(size_t)act[b0 + (size_t)k]];
                N3_CALL(product(eg.key, jobs.job[2 * k].x, jobs.job[2 * k].y, st));
                N3_CALL(product(eg.value, jobs.job[2 * k + 1].x, jobs.job[2 * k + 1].y, st));
            }
        }
        if (conv) {
            rn_launch(n3_engram_conv_kernel, dim3((d + 255) / 256, 1, ns), dim3(256), 0, st, cs, position, keep,
                      (int)g.engram_conv_taps, (int)g.engram_conv_dilation, d, 1);
            N3_HIP(hipGetLastError());
        }
    }
    return RN_OK;
}

// The probe heads observe the cells of `count` tokens in order (heads.rs:138-155),
// kN3MaxHeads heads a launch
int enqueue_observe(rn_n3_session* s, const float* cells, int cell_stride, int count) {
    const rn_n3_model* m = s->m;
    hipStream_t st = s->stream;
    for (size_t b0 = 0; b0 < m->heads.size(); b0 += kN3MaxHeads) {
        if (count > 1) {
            for (size_t i = b0; i < std::min(m->heads.size(), b0 + kN3MaxHeads); ++i) {
                const N3Head& h = m->heads[i];
                rn_launch(n3_observe_run_kernel, dim3(h.layers * h.per_layer), dim3(256), 0, st, cells, cell_stride,
                          count, (const float*)h.probes, h.per_layer, h.width, s->peak[i], s->total[i],
                          s->weighted[i]);
                N3_HIP(hipGetLastError());
            }
            continue;
        }
        N3ObserveHeads hs{};
        int blocks = 0;
        for (size_t i = b0; i < std::min(m->heads.size(), b0 + kN3MaxHeads); ++i) {
            const N3Head& h = m->heads[i];
            const int k = hs.count++;
            hs.probes[k] = h.probes;
            hs.peak[k] = s->peak[i];
            hs.total[k] = s->total[i];
            hs.weighted[k] = s->weighted[i];
            hs.k[k] = h.per_layer;
            hs.width[k] = h.width;
            hs.first[k] = blocks;
            blocks += h.layers * h.per_layer;
        }
        hs.first[hs.count] = blocks;
        rn_launch(n3_observe_kernel, dim3(blocks), dim3(256), 0, st, cells, hs);
        N3_HIP(hipGetLastError());
    }
    return RN_OK;
}

// Session::push (session.rs:76-148) of tokens[position], which the host writes
// (source null) or a device value (source: the greedy argmax) supplies.
int enqueue_push(rn_n3_session* s, uint32_t token, const uint32_t* source) {
    const rn_n3_model* m = s->m;
    const rn_geometry& g = m->g;
    const int d = (int)g.d_model, lanes = (int)g.mhc_lanes;
    const int position = s->length;
    float* cur = s->stream_a;
    float* nxt = s->stream_b;
    // the embedding (session.rs:86-97) and the engram sites (engram.rs:30-112)
    // before the layers: one launch embeds the token and gathers and prepares
    // the active sites' inputs, one runs their key and value products, one
    // their value convolutions (the fused layers convolve in their boundary)
    N3GatherSites em{};
    em.embed = 1;
    em.table = m->embedding->cb;
    em.tokens = s->tokens_dev;
    em.position = position;
    em.d = d;
    em.lanes = lanes;
    em.scale = sqrtf((float)d);
    em.stream = cur;
    em.cell = s->cells;
    em.source = source;
    em.value = token;
    N3_CALL(enqueue_sites(s, position, !s->fused, &em));

    N3_CALL(s->fused ? fused_layers(s, position, cur, nxt) : stepwise_layers(s, position, cur, nxt));
    s->lrot_ready = s->fused;
    N3_CALL(enqueue_observe(s, s->cells, 0, 1));
    s->length++;
    return RN_OK;
}

// Session::logits (session.rs:151-165) into s->logits on the device
int enqueue_logits(rn_n3_session* s) {
    const rn_n3_model* m = s->m;
    hipStream_t st = s->stream;
    const float* in = s->lrot;
    if (!s->lrot_ready) {
        rn_launch(n3_fake_quantise_kernel, dim3(1), dim3(kN3Block), 0, st, (const float*)s->hidden, (int)m->g.d_model,
                  m->embedding->cb.padded, m->embedding->group, m->embedding->cb.wht_scale, s->rotated);
        N3_HIP(hipGetLastError());
        in = s->rotated;
    }
    CodebookParams p = m->embedding->cb;
    p.rows = m->output_vocab;  // multiply_rows(0, ..) over the first output_vocab rows
    if (m->embedding->bits == 1 || m->embedding->bits == 3)
        N3_HIP(launch_codebook_float(p, in, 1, s->logits, false, st));
    else
        N3_HIP(launch_codebook_product(p, in, 1, s->logits, nullptr, st));
    return RN_OK;
}

// The vectors of a batched feed, once a session
int run_buffers(rn_n3_session* s) {
    rn_n3_session::Run& r = s->run;
    if (r.ready) return RN_OK;
    const rn_n3_model* m = s->m;
    const rn_geometry& g = m->g;
    const size_t C = kN3FeedChunk, d = g.d_model, S = (size_t)g.mhc_lanes * d, H = g.num_heads;
    const size_t A = m->active.size();
    size_t widest = 0, rows = 0, gathered = 1;
    for (const N3Layer& y : m->layers) {
        widest = std::max({widest, (size_t)y.qkvg->cb.padded, (size_t)y.out->cb.padded});
        rows = std::max(rows, (size_t)y.qkvg->rows);
    }
    for (const N3Engram& e : m->engrams) {
        widest = std::max(widest, (size_t)e.key->cb.padded);
        gathered = std::max(gathered, (size_t)e.key->columns);
    }
    N3_CALL(alloc_n(s, C * S, &r.stream_a));
    N3_CALL(alloc_n(s, C * S, &r.stream_b));
    N3_CALL(alloc_n(s, C * d, &r.attn));
    N3_CALL(alloc_n(s, C * d, &r.x));
    N3_CALL(alloc_n(s, C * d, &r.input));
    N3_CALL(alloc_n(s, C * kMaxLanes, &r.post));
    N3_CALL(alloc_n(s, C * kMaxLanes * kMaxLanes, &r.residual));
    N3_CALL(alloc_n(s, C * widest, &r.rotated));
    N3_CALL(alloc_n(s, C * rows, &r.prod));
    N3_CALL(alloc_n(s, C * H * 64, &r.attended));
    N3_CALL(alloc_n(s, C * H * 64, &r.qcodes));
    N3_CALL(alloc_n(s, C * H, &r.qscales));
    N3_CALL(alloc_n(s, C * (A + 1) * d, &r.cells));
    N3_CALL(alloc_n(s, C * gathered, &r.gathered));
    N3_CALL(alloc_n(s, C * d, &r.eraw));
    r.ekey.assign(g.engram_site_count, nullptr);
    r.evalue.assign(g.engram_site_count, nullptr);
    for (uint32_t e = 0; e < g.engram_site_count; ++e) {
        N3_CALL(alloc_n(s, C * d, &r.ekey[e]));
        N3_CALL(alloc_n(s, C * d, &r.evalue[e]));
    }
    r.ready = true;
    return RN_OK;
}

// Session::prefill (prefill.rs:10-99) of count (<= kN3FeedChunk) tokens at
// positions [length, length + count): the per-token work of a layer runs as
// one launch over the tokens (a block or a grid row each), the projections as
// batched products, the attention per (head, token) after every token's key
// and value joined the cache; each token's arithmetic is the push's, so the
// state after the run equals that after pushing the tokens in order.
int enqueue_run(rn_n3_session* s, const uint32_t* tokens, int count) {
    N3_CALL(run_buffers(s));
    const rn_n3_model* m = s->m;
    const rn_geometry& g = m->g;
    rn_n3_session::Run& r = s->run;
    const int d = (int)g.d_model, lanes = (int)g.mhc_lanes, H = (int)g.num_heads, KV = (int)g.num_kv_heads;
    const int S = lanes * d, T = count, P0 = s->length;
    const size_t layers = m->active.size();
    const int cell_stride = (int)(layers + 1) * d;
    hipStream_t st = s->stream;
    {
        N3TokenRun ids{};
        for (int i = 0; i < T; ++i) ids.ids[i] = tokens[i];
        rn_launch(n3_set_tokens_kernel, dim3(1), dim3(256), 0, st, s->tokens_dev, P0, T, ids);
        N3_HIP(hipGetLastError());
    }
    const int embed_threads = ((m->embedding->cb.padded / 16 + 63) / 64) * 64;
    rn_launch(n3_embed_kernel, dim3(T), dim3(embed_threads), 0, st, m->embedding->cb, s->tokens_dev, P0, d, lanes,
              sqrtf((float)d), r.stream_a, r.cells, S, cell_stride, 0, (const uint32_t*)nullptr, 0u);
    N3_HIP(hipGetLastError());

    // engram sites (engram.rs:113-162)
    const int hpo = heads_per_order(g), tables = (int)g.engram_order_count * hpo;
    const int keep = std::max(1, ((int)g.engram_conv_taps - 1) * (int)g.engram_conv_dilation + 1);
    for (uint32_t e = 0; e < g.engram_site_count; ++e) {
        if (!site_active(m, (int)e)) continue;
        const N3Engram& eg = m->engrams[e];
        N3GatherParams gp{};
        gp.tables = eg.tables->cb;
        gp.count = tables;
        gp.sub = (int)g.engram_sub_dim;
        gp.slots = (int)g.engram_slots;
        gp.position = P0;
        gp.tokens = s->tokens_dev;
        gp.heads_per_order = hpo;
        gp.stride = g.engram_seed_heads == 0 ? hpo : (int)g.engram_seed_heads;
        for (int o = 0; o < 4; ++o) gp.orders[o] = (int)g.engram_orders[o];
        gp.out = r.gathered;
        gp.out_stride = (int)eg.key->columns;
        N3GatherSites gs{};
        gs.site[0] = gp;
        rn_launch(n3_gather_kernel, dim3(T, 1), dim3(kN3Block), 0, st, gs);
        N3_HIP(hipGetLastError());
        N3_HIP(launch_codebook_rotate(r.gathered, T, eg.key->columns, eg.key->cb.padded, eg.key->group,
                                      eg.key->cb.wht_scale, r.rotated, st));
        N3_CALL(product_run(eg.key, r.rotated, T, r.ekey[e], st));
        N3_CALL(product_run(eg.value, r.rotated, T, r.eraw, st));
        N3ConvSites cs{};
        cs.raw[0] = r.eraw;
        cs.ring[0] = s->rings[e];
        cs.taps[0] = eg.taps;
        cs.value[0] = r.evalue[e];
        rn_launch(n3_engram_conv_kernel, dim3((d + 255) / 256, T, 1), dim3(256), 0, st, cs, P0, keep,
                  (int)g.engram_conv_taps, (int)g.engram_conv_dilation, d, 0);
        N3_HIP(hipGetLastError());
        rn_launch(n3_ring_store_kernel, dim3((d + 255) / 256, std::min(T, keep)), dim3(256), 0, st, (const float*)r.eraw,
                  d, T, P0, keep, d, s->rings[e], d);
        N3_HIP(hipGetLastError());
    }

    float* cur = r.stream_a;
    float* nxt = r.stream_b;
    auto route_into = [&](N3BoundaryParams& b, size_t slot) {
        const int layer = m->active[slot];
        const N3Layer& y = m->layers[(size_t)layer];
        const int site = site_of(m, layer);
        b.route = 1;
        b.layer = layer;
        b.slot = (int)slot;
        b.phi_pre = m->phi_pre->cb;
        b.phi_post = m->phi_post->cb;
        b.phi_res = m->phi_res->cb;
        b.a_pre = m->a_pre;
        b.a_post = m->a_post;
        b.a_res = m->a_res;
        b.b_pre = m->b_pre;
        b.b_post = m->b_post;
        b.b_res = m->b_res;
        b.input = r.input;
        b.post = r.post;
        b.residual = r.residual;
        b.key = site >= 0 ? r.ekey[(size_t)site] : nullptr;
        b.value = site >= 0 ? r.evalue[(size_t)site] : nullptr;
        b.norm_in = y.norm_in;
        b.x = r.x;
        b.qpadded = y.qkvg->cb.padded;
        b.qgroup = y.qkvg->group;
        b.qib = y.qkvg->bits == 5 ? 2 : y.qkvg->bits;
        b.qscale = y.qkvg->cb.wht_scale;
        b.rotated = r.rotated;
        b.phi_rows = m->phi_stack + (size_t)layer * (2 * lanes + lanes * lanes) * m->phi_pre->cb.row_bytes;
    };
    {
        N3BoundaryParams b{};
        b.stream = cur;
        b.d = d;
        b.lanes = lanes;
        b.cell_stride = cell_stride;
        route_into(b, 0);
        rn_launch(n3_boundary_kernel, dim3(T), dim3(kN3Block), 0, st, b);
        N3_HIP(hipGetLastError());
    }
    const int qw = H * 64, qkv = (H + 2 * KV) * 64;
    for (size_t slot = 0; slot < layers; ++slot) {
        const int layer = m->active[slot];
        const N3Layer& y = m->layers[(size_t)layer];
        N3CacheDev& c = s->caches[(size_t)layer];
        const int rows = (int)y.qkvg->rows;
        N3_CALL(product_run(y.qkvg, r.rotated, T, r.prod, st));
        N3QkvParams qp{};
        qp.prod = r.prod;
        qp.hist = c.hist;
        for (int t = 0; t < 3; ++t) qp.taps[t] = y.taps[t];
        qp.ntaps = (int)g.qkv_conv_taps;
        qp.position = P0;
        qp.H = H;
        qp.KV = KV;
        qp.cap = s->capacity;
        qp.q_norm = y.q_norm;
        qp.k_norm = y.k_norm;
        qp.cos_row = s->cos + (size_t)P0 * 32;
        qp.sin_row = s->sin + (size_t)P0 * 32;
        qp.qcodes = r.qcodes;
        qp.qscales = r.qscales;
        qp.keys = c.keys;
        qp.key_scales = c.key_scales;
        qp.values = c.values;
        qp.value_scales = c.value_scales;
        qp.prod_stride = rows;
        qp.run = 1;
        rn_launch(n3_qkv_kernel, dim3(H + 2 * KV, T), dim3(64), 0, st, qp);
        N3_HIP(hipGetLastError());
        if (qp.ntaps > 0) {
            rn_launch(n3_ring_store_kernel, dim3((qkv + 255) / 256, std::min(T, qp.ntaps)), dim3(256), 0, st,
                      (const float*)r.prod, rows, T, P0, qp.ntaps, qkv, c.hist, qkv);
            N3_HIP(hipGetLastError());
        }
        N3AttendParams ap{r.qcodes, r.qscales, c.keys, c.key_scales, c.values, c.value_scales, r.prod + qkv,
                          s->capacity, P0, layer_window(g, layer), H / KV, 1.0f / sqrtf(64.0f), r.attended, rows};
        rn_launch(n3_attend_kernel, dim3(H, T), dim3(256), 0, st, ap);
        N3_HIP(hipGetLastError());
        rn_launch(n3_fake_quantise_kernel, dim3(T), dim3(kN3Block), 0, st, (const float*)r.attended, qw,
                  y.out->cb.padded, y.out->group, y.out->cb.wht_scale, r.rotated);
        N3_HIP(hipGetLastError());
        N3_CALL(product_run(y.out, r.rotated, T, r.attn, st));
        N3BoundaryParams b{};
        b.tail = 1;
        N3BlockOutParams& bo = b.t;
        bo.attention = r.attn;
        bo.post_norm = y.post_norm;
        bo.gate = y.gate_sigmoid;
        bo.pre_norm = y.pre_norm;
        bo.d1 = y.d1;
        bo.d2 = y.d2;
        bo.b2 = y.b2;
        bo.d3 = y.d3;
        bo.d4 = y.d4;
        for (int f = 0; f < 6; ++f) bo.factors[f] = y.factors[f];
        bo.cond_v = y.cond_v;
        bo.cond_u = y.cond_u;
        bo.rank = y.rank;
        bo.perm1 = m->perm[0];
        bo.perm2 = m->perm[1];
        bo.x = r.x;
        bo.input = r.input;
        bo.post = r.post;
        bo.residual = r.residual;
        bo.stream = cur;
        bo.d = d;
        bo.lanes = lanes;
        bo.next = nxt;
        bo.cell = r.cells + (slot + 1) * (size_t)d;
        b.d = d;
        b.lanes = lanes;
        b.cell_stride = cell_stride;
        if (slot + 1 < layers) {
            route_into(b, slot + 1);
        } else {
            b.final = 1;
            b.final_norm = m->final_norm;
            b.hidden = s->hidden;
        }
        rn_launch(n3_boundary_kernel, dim3(T), dim3(kN3Block), 0, st, b);
        N3_HIP(hipGetLastError());
        std::swap(cur, nxt);
    }
    // the heads observe the tokens in order (prefill.rs:92-96)
    N3_CALL(enqueue_observe(s, r.cells, cell_stride, T));
    // the last token's cells (prefill.rs:98)
    N3_HIP(hipMemcpyAsync(s->cells, r.cells + (size_t)(T - 1) * cell_stride, (size_t)cell_stride * 4,
                          hipMemcpyDeviceToDevice, st));
    s->length += T;
    s->lrot_ready = false;
    return RN_OK;
}

// A run of tokens can take the batched path: the one-launch boundary and
// vectors on 16-byte boundaries (its products take either path, so float-path
// projections run it too); RN_N3_PATH=stepwise keeps every token a push.
bool run_applies(const rn_n3_session* s) {
    const rn_n3_model* m = s->m;
    const rn_geometry& g = m->g;
    const int d = (int)g.d_model;
    const char* path = getenv("RN_N3_PATH");
    if ((path && strcmp(path, "stepwise") == 0) || !boundary_applies(m) || m->phi_stack == nullptr || d % 4 != 0)
        return false;
    for (const N3Head& h : m->heads)
        if (h.width != d) return false;
    const int gathered = (int)(g.engram_order_count * heads_per_order(g) * g.engram_sub_dim);
    for (const N3Engram& e : m->engrams)
        if ((int)e.key->columns != gathered || (int)e.key->rows != d || (int)e.value->rows != d) return false;
    for (const N3Layer& y : m->layers)
        if ((int)y.out->rows != d || (int)y.qkvg->rows < ((int)g.num_heads * 2 + 2 * (int)g.num_kv_heads) * 64)
            return false;
    return true;
}

}  // namespace

int rn_n3_session_push(rn_n3_session* s, uint32_t token) {
    N3_REQUIRE(s, "null session");
    N3_REQUIRE(token < s->m->g.vocab, "token %u is outside the vocabulary of %u", token, s->m->g.vocab);
    N3_REQUIRE(s->length < s->capacity, "session is full (capacity %d)", s->capacity);
    return enqueue_push(s, token, nullptr);
}

// Generator::run_turn's greedy loop (generator.rs:199-230, argmax at 257-265)
// without grammar: token = first; `steps` times { push(token); logits; token =
// argmax; ids[i] = token }. The argmax stays on the device and feeds the next
// push; the host waits once, for the ids.
int rn_n3_session_decode_greedy(rn_n3_session* s, uint32_t first, int steps, uint32_t* ids) {
    N3_REQUIRE(s && (ids || steps == 0), "null argument");
    N3_REQUIRE(steps >= 0, "steps must be non-negative");
    N3_REQUIRE(first < s->m->g.vocab, "token %u is outside the vocabulary of %u", first, s->m->g.vocab);
    N3_REQUIRE(s->length + steps <= s->capacity, "%d steps overflow the capacity", steps);
    if (steps == 0) return RN_OK;
    N3_REQUIRE(steps <= s->capacity, "steps above the capacity");
    for (int i = 0; i < steps; ++i) {
        N3_CALL(enqueue_push(s, first, i == 0 ? nullptr : s->next_dev));
        N3_CALL(enqueue_logits(s));
        N3_HIP(launch_argmax_rows(s->logits, 1, s->m->output_vocab, s->next_dev, s->ids_dev, steps, i, s->stream));
    }
    N3_HIP(hipMemcpyAsync(ids, s->ids_dev, (size_t)steps * 4, hipMemcpyDeviceToHost, s->stream));
    N3_HIP(hipStreamSynchronize(s->stream));
    return RN_OK;
}

// #[derive(Clone)] on Session (session.rs:17), the Generator's prefix cache
// (generator.rs:41-46: the base session with the system prompt is cloned per
// turn and on reset). A new session of the same capacity takes its chunks in
// the same order, so every buffer sits at the same offset of the same chunk;
// copying the chunks copies the whole state (caches, conv and engram rings,
// lanes stream, token history, cells, probe-head accumulators, hidden state
// and logits' input). No session buffer holds a device pointer.
int rn_n3_session_clone(const rn_n3_session* s, rn_n3_session** out) {
    N3_REQUIRE(s && out, "null argument");
    *out = nullptr;
    rn_n3_session* t = nullptr;
    N3_CALL(rn_n3_session_create(s->m, s->capacity, &t));
    auto fail_with = [&](int rc) {
        rn_n3_session_free(t);
        return rc;
    };
    t->fused = s->fused;
    if (s->run.ready) {
        const int rc = run_buffers(t);
        if (rc) return fail_with(rc);
    }
    if (t->allocation_bytes != s->allocation_bytes)
        return fail_with(n3_fail(RN_ERR_STATE, "the clone's buffers do not line up with the session's"));
    hipError_t e = hipStreamSynchronize(s->stream);
    for (size_t i = 0; i < s->allocations.size() && e == hipSuccess; ++i)
        e = hipMemcpyAsync(t->allocations[i], s->allocations[i], s->allocation_bytes[i], hipMemcpyDeviceToDevice,
                           t->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(t->stream);
    if (e != hipSuccess) return fail_with(n3_fail(RN_ERR_DEVICE, "clone: %s", hipGetErrorString(e)));
    t->length = s->length;
    t->lrot_ready = s->lrot_ready;
    *out = t;
    return RN_OK;
}

// The loop of Generator::run_turn (generator.rs:99-130) with no grammar active:
//   while n < max_tokens && len + 1 < window { next = argmax(logits);
//     ids[n++] = next; push(next); if next is a stop token { finished; break } }
// The logits, argmax and push stay on the device (the push reads the argmax
// there). The host learns each token while the push of it runs: the next
// token's logits and argmax are queued before the host waits for the
// previous token, so the device never waits for the stop test. A stop token
// is pushed, nothing after it. *count gets n, *finished 1 after a stop token.
int rn_n3_session_run_turn(rn_n3_session* s, int max_tokens, int window, const uint32_t* stops, int stop_count,
                           uint32_t* ids, int* count, int* finished) {
    N3_REQUIRE(s && count && finished && (ids || max_tokens == 0) && (stops || stop_count == 0), "null argument");
    N3_REQUIRE(max_tokens >= 0 && stop_count >= 0, "max_tokens and stop_count must be non-negative");
    *count = 0;
    *finished = 0;
    N3_REQUIRE(s->length > 0, "no token has been pushed (the turn's logits need one)");
    if (window <= 0) window = (int)s->m->g.max_seq_len;  // ModelConfig::max_seq_len, as run_turn takes it
    const int room = std::max(0, std::min(max_tokens, window - 1 - s->length));
    N3_REQUIRE(s->length + room <= s->capacity, "a turn of up to %d tokens overflows the capacity %d", room,
               s->capacity);
    if (room == 0) return RN_OK;
    if (!s->turn_host) {
        N3_HIP(hipHostMalloc((void**)&s->turn_host, 2 * sizeof(uint32_t), hipHostMallocDefault));
        for (hipEvent_t& e : s->turn_done) N3_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    }
    hipStream_t st = s->stream;
    // the logits of the state after n pushes, the argmax into next_dev and
    // ids_dev[n], its copy to the host slot n % 2
    auto choose = [&](int n) -> int {
        N3_CALL(enqueue_logits(s));
        N3_HIP(launch_argmax_rows(s->logits, 1, s->m->output_vocab, s->next_dev, s->ids_dev, room, n, st));
        N3_HIP(hipMemcpyAsync(s->turn_host + (n & 1), s->next_dev, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
        N3_HIP(hipEventRecord(s->turn_done[n & 1], st));
        return RN_OK;
    };
    N3_CALL(choose(0));
    int n = 0;
    while (n < room) {
        N3_CALL(enqueue_push(s, 0, s->next_dev));
        ++n;
        if (n < room) N3_CALL(choose(n));
        N3_HIP(hipEventSynchronize(s->turn_done[(n - 1) & 1]));
        const uint32_t token = s->turn_host[(n - 1) & 1];
        if (std::find(stops, stops + stop_count, token) != stops + stop_count) {
            *finished = 1;
            break;
        }
    }
    N3_HIP(hipMemcpyAsync(ids, s->ids_dev, (size_t)n * 4, hipMemcpyDeviceToHost, st));
    N3_HIP(hipStreamSynchronize(st));
    *count = n;
    return RN_OK;
}

// generator.rs:104-116 while a tool-call grammar is active: the session's
// logits (Session::logits), argmax_allowed over the host's mask with the
// argmax fallback, and allowed_statistics of the choice, on the device.
int rn_n3_session_choose_allowed(rn_n3_session* s, const uint8_t* allowed, rn_choice* out) {
    N3_REQUIRE(s && allowed && out, "null argument");
    N3_REQUIRE(s->length > 0, "no token has been pushed");
    static_assert(sizeof(rn_choice) == sizeof(Choice), "rn_choice mirrors rn::Choice");
    const int n = s->m->output_vocab;
    N3_CALL(enqueue_logits(s));
    N3_HIP(hipMemcpyAsync(s->allowed_dev, allowed, (size_t)n, hipMemcpyHostToDevice, s->stream));
    N3_HIP(launch_constrained_choice(s->logits, s->allowed_dev, n, -1, s->choice_dev, s->stream));
    N3_HIP(hipMemcpyAsync(out, s->choice_dev, sizeof(Choice), hipMemcpyDeviceToHost, s->stream));
    N3_HIP(hipStreamSynchronize(s->stream));
    return RN_OK;
}

// Session::feed (session.rs:58-74): at least BATCH_THRESHOLD (4) tokens run
// as batched prefills (a shorter last chunk of fewer than 4 is pushed), fewer
// are pushed. With integer-path engram matrices the batched prefill runs each
// token's arithmetic as a push does, so the chunk size changes nothing but
// speed, and runs take up to kN3FeedChunk tokens (RN_N3_FEED_CHUNK, 4..256,
// sets it). A 1- or 3-bit projection, engram key or engram value matrix takes
// the float path, whose batch tile (multiply_batch, matrix.rs:330-389) rounds
// differently from its vector path: then the chunks are the reference's
// PREFILL_CHUNK of 128 (session.rs:11), so that the same tokens run batched
// and pushed as there.
int rn_n3_session_feed(rn_n3_session* s, const uint32_t* tokens, int count) {
    constexpr int kBatchThreshold = 4, kPrefillChunk = 128;
    N3_REQUIRE(s && (tokens || count == 0), "null argument");
    N3_REQUIRE(count >= 0 && s->length + count <= s->capacity, "feed of %d tokens overflows the capacity", count);
    for (int i = 0; i < count; ++i) N3_REQUIRE(tokens[i] < s->m->g.vocab, "token %u outside the vocabulary", tokens[i]);
    // the products whose batch arithmetic differs from their vector arithmetic
    // (1- and 3-bit matrices: multiply_batch's float tile, matrix.rs:356-378):
    // the projections (attend_batch) and the engram key and value
    // (contribute_batch); then the runs are the reference's chunks
    bool float_batch = false;
    for (const N3Engram& e : s->m->engrams) float_batch |= !integer_path(e.key) || !integer_path(e.value);
    for (int layer : s->m->active) {
        const N3Layer& y = s->m->layers[(size_t)layer];
        float_batch |= !integer_path(y.out) || (y.qkvg != nullptr && !integer_path(y.qkvg));
    }
    int chunk = float_batch ? kPrefillChunk : kN3FeedChunk;
    if (const char* e = getenv("RN_N3_FEED_CHUNK"))
        if (!float_batch) chunk = std::min(kN3FeedChunk, std::max(kBatchThreshold, atoi(e)));
    if (count < kBatchThreshold || !run_applies(s)) {
        for (int i = 0; i < count; ++i) N3_CALL(rn_n3_session_push(s, tokens[i]));
        return RN_OK;
    }
    for (int i = 0; i < count; i += chunk) {
        const int n = std::min(chunk, count - i);
        if (n >= kBatchThreshold) {
            N3_CALL(enqueue_run(s, tokens + i, n));
        } else {
            for (int j = 0; j < n; ++j) N3_CALL(rn_n3_session_push(s, tokens[i + j]));
        }
    }
    return RN_OK;
}

int rn_n3_session_length(const rn_n3_session* s, int* length) {
    N3_REQUIRE(s && length, "null argument");
    *length = s->length;
    return RN_OK;
}

// Session::logits (session.rs:151-165): logits [output_vocab] on the host
int rn_n3_session_logits(rn_n3_session* s, float* logits) {
    N3_REQUIRE(s && logits, "null argument");
    N3_CALL(enqueue_logits(s));
    N3_HIP(hipMemcpyAsync(logits, s->logits, (size_t)s->m->output_vocab * 4, hipMemcpyDeviceToHost, s->stream));
    N3_HIP(hipStreamSynchronize(s->stream));
    return RN_OK;
}

int rn_n3_session_hidden(rn_n3_session* s, float* hidden) {
    N3_REQUIRE(s && hidden, "null argument");
    N3_HIP(hipMemcpyAsync(hidden, s->hidden, (size_t)s->m->g.d_model * 4, hipMemcpyDeviceToHost, s->stream));
    N3_HIP(hipStreamSynchronize(s->stream));
    return RN_OK;
}

// Session::cells (session.rs:137-139): [active + 1][d_model] of the last push
int rn_n3_session_cells(rn_n3_session* s, float* cells) {
    N3_REQUIRE(s && cells, "null argument");
    const size_t n = (s->m->active.size() + 1) * (size_t)s->m->g.d_model;
    N3_HIP(hipMemcpyAsync(cells, s->cells, n * 4, hipMemcpyDeviceToHost, s->stream));
    N3_HIP(hipStreamSynchronize(s->stream));
    return RN_OK;
}

namespace {
int pooled_into(rn_n3_session* s, size_t i) {
    const N3Head& h = s->m->heads[i];
    const int slots = h.layers * h.per_layer;
    rn_launch(n3_readout_kernel, dim3(slots), dim3(256), 0, s->stream, (const float*)s->weighted[i],
              (const float*)s->total[i], (const float*)h.gain, h.width, s->readouts);
    N3_HIP(hipGetLastError());
    rn_launch(n3_pool_kernel, dim3(h.queries), dim3(256), 0, s->stream, (const float*)s->readouts, slots,
              (const float*)h.query, (const float*)h.row_bias, h.width, s->pooled);
    N3_HIP(hipGetLastError());
    return RN_OK;
}
int head_index(const rn_n3_model* m, int code) {
    for (size_t i = 0; i < m->heads.size(); ++i)
        if (m->heads[i].code == code) return (int)i;
    return -1;
}
}  // namespace

// Session::pooled_readout (session.rs:131-135; heads.rs:99-125): queries x width
// floats on the host; *count is 0 when no head has the code.
int rn_n3_session_pooled_readout(rn_n3_session* s, int code, float* out, int capacity, int* count) {
    N3_REQUIRE(s && count, "null argument");
    const int i = head_index(s->m, code);
    *count = 0;
    if (i < 0) return RN_OK;
    const N3Head& h = s->m->heads[(size_t)i];
    N3_REQUIRE(s->length > 0, "no token has been observed");
    const int n = h.queries * h.width;
    N3_REQUIRE(out && capacity >= n, "output holds %d floats, %d needed", capacity, n);
    N3_CALL(pooled_into(s, (size_t)i));
    N3_HIP(hipMemcpyAsync(out, s->pooled, (size_t)n * 4, hipMemcpyDeviceToHost, s->stream));
    N3_HIP(hipStreamSynchronize(s->stream));
    *count = n;
    return RN_OK;
}

// Session::head_output (session.rs:125-129; heads.rs:127-136)
int rn_n3_session_head_output(rn_n3_session* s, int code, float* out, int capacity, int* count) {
    N3_REQUIRE(s && count, "null argument");
    const int i = head_index(s->m, code);
    *count = 0;
    if (i < 0) return RN_OK;
    const N3Head& h = s->m->heads[(size_t)i];
    N3_REQUIRE(s->length > 0, "no token has been observed");
    const int rows = h.projection->rows;
    N3_REQUIRE(out && capacity >= rows, "output holds %d floats, %d needed", capacity, rows);
    N3_CALL(pooled_into(s, (size_t)i));
    N3_CALL(rotate(h.projection, s->pooled, s->rotated, s->stream));
    N3_CALL(product(h.projection, s->rotated, s->head_out, s->stream));
    rn_launch(n3_add_kernel, dim3((rows + 255) / 256), dim3(256), 0, s->stream, s->head_out, (const float*)h.bias, rows);
    N3_HIP(hipGetLastError());
    N3_HIP(hipMemcpyAsync(out, s->head_out, (size_t)rows * 4, hipMemcpyDeviceToHost, s->stream));
    N3_HIP(hipStreamSynchronize(s->stream));
    *count = rows;
    return RN_OK;
}

// The int8 cache of one layer for the first `length` positions, on the host:
// keys / values [length][kv][64] (the reference's order), scales [kv][length].
int rn_n3_session_cache(rn_n3_session* s, int layer, int8_t* keys, float* key_scales, int8_t* values,
                        float* value_scales) {
    N3_REQUIRE(s && keys && key_scales && values && value_scales, "null argument");
    N3_REQUIRE(layer >= 0 && layer < (int)s->m->g.num_layers, "layer %d out of range", layer);
    // the cache of a layer outside the ladder's selection stays empty in the
    // reference (session.rs:99-101 never visits it): refuse it here
    N3_REQUIRE(std::find(s->m->active.begin(), s->m->active.end(), layer) != s->m->active.end(),
               "layer %d is not an active layer at this depth", layer);
    const int KV = (int)s->m->g.num_kv_heads, n = s->length, cap = s->capacity;
    const N3CacheDev& c = s->caches[(size_t)layer];
    std::vector<int8_t> k((size_t)KV * cap * 64), v(k.size());
    std::vector<float> ks((size_t)KV * cap), vs(ks.size());
    N3_HIP(hipStreamSynchronize(s->stream));
    N3_HIP(hipMemcpy(k.data(), c.keys, k.size(), hipMemcpyDeviceToHost));
    N3_HIP(hipMemcpy(v.data(), c.values, v.size(), hipMemcpyDeviceToHost));
    N3_HIP(hipMemcpy(ks.data(), c.key_scales, ks.size() * 4, hipMemcpyDeviceToHost));
    N3_HIP(hipMemcpy(vs.data(), c.value_scales, vs.size() * 4, hipMemcpyDeviceToHost));
    for (int p = 0; p < n; ++p)
        for (int h = 0; h < KV; ++h) {
            memcpy(keys + ((size_t)p * KV + h) * 64, k.data() + ((size_t)h * cap + p) * 64, 64);
            memcpy(values + ((size_t)p * KV + h) * 64, v.data() + ((size_t)h * cap + p) * 64, 64);
        }
    for (int h = 0; h < KV; ++h) {
        memcpy(key_scales + (size_t)h * n, ks.data() + (size_t)h * cap, (size_t)n * 4);
        memcpy(value_scales + (size_t)h * n, vs.data() + (size_t)h * cap, (size_t)n * 4);
    }
    return RN_OK;
}

int rn_n3_session_stream(const rn_n3_session* s, void** stream) {
    N3_REQUIRE(s && stream, "null argument");
    *stream = s->stream;
    return RN_OK;
}
