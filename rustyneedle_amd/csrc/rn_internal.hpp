// rn_internal.hpp — launch descriptors shared between the kernel translation
// units and the C-ABI layer (rn_api.hip). Plain structs passed by value as
// kernel arguments.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace rn {

// Launch hook of the per-kernel profiler: when a pair of events is armed, the
// next launch records them around the kernel's own execution
// (hipExtLaunchKernelGGL), so the interval excludes queueing gaps.
struct LaunchEvents {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};
LaunchEvents& launch_events();  // per host thread

// Records `message` as the calling thread's last error (rn_last_error); returns `code`.
int set_error(int code, const char* message);

template <typename F, typename... Args>
inline void rn_launch(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream, Args... args) {
    LaunchEvents& ev = launch_events();
    if (ev.start != nullptr) {
        hipEvent_t start = ev.start, stop = ev.stop;
        ev.start = ev.stop = nullptr;
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, stream, start, stop, 0u, args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
    }
}

constexpr int kGroup = 32;  // int8 codes per fp32 weight scale

// Per-session decode state in device memory. The greedy step reads `token`,
// the attention kernels read `pos`, the argmax finalize kernel writes the next
// token back into `token` and `ids[step]`.
struct DecodeState {
    uint32_t token;
    int32_t pos;
    uint32_t step;
    int32_t error;
    uint32_t ids_capacity;
};

// kClassSum: the input is 32 partial vectors [32][K] (the per-class value sums
// of the decoder's cross-attention), added in class order 0..31 before the
// quantisation of kQuant. kCrossNorm: the cross-attention residual first
// (x + cross_gain * zero_centred_norm(attended, post_gain), cross.rs:176-181;
// block 0 writes it to x_out), then kNorm on that sum.
// kEmbedArgmax (the batch-1 head kernel only): the token is the greedy choice
// of the previous step's logits, reduced from the logits kernel's block keys.
enum GemvPrologue { kQuant = 0, kNorm = 1, kEmbedNorm = 2, kCodes = 3, kClassSum = 4, kCrossNorm = 5, kEmbedArgmax = 6 };
enum GemvEpilogue { kStore = 0, kResidual = 1, kSilu = 2, kArgmax = 3 };
enum ProductForm { kPanel = 0, kPlane = 1 };

// One matrix of a (possibly fused) batch-1 product launch.
struct Segment {
    const int8_t* W;   // [rows][K]
    const float* sW;   // [rows][K/32]
    float* y;          // store target (kStore/kSilu/kArgmax) or residual x (kResidual)
    int32_t* acc;      // nullable [rows][K/32]
    int rows;          // rows of W (kSilu: 2*half_rows)
};
constexpr int kMaxSegments = 8;
static_assert(sizeof(Segment) == 40, "the first segment, after 24 leading bytes, ends the first 64-byte line");

// The prologue's input and the first segment share the first 64 bytes of the
// argument segment (one scalar-cache line). Segment s is grid row y = s, so a
// block reads its segment at an address known when it starts: it requests its
// input vector and its weights after one argument load.
struct GemvParams {
    const float* x;       // input vector (kQuant/kNorm)
    const float* gain;    // zero-centred norm gains (kNorm/kEmbedNorm)
    int nseg;
    int half_rows;        // kSilu: ffn width (gate rows 0..half-1, up rows half..2*half-1)
    Segment seg[kMaxSegments];
    const float* attended;     // kCrossNorm: the cross-attention output and its post-norm gains
    const float* post_gain;
    DecodeState* state;   // kEmbedNorm: the token to embed
    float eps;
    float cross_gain;
    const int8_t* xq;     // kCodes: pre-quantised input
    const float* xs;
    const int8_t* embW;   // kEmbedNorm: embedding codes/scales, the token comes from state
    const float* embS;
    float embed_scale;    // sqrt(d_model)
    int vocab;
    float* x_out;         // kEmbedNorm / kCrossNorm: block 0 writes the new residual row
    float* hidden_out;    // kNorm: block 0 writes the normed input (nullable)
    unsigned long long* keys;  // kArgmax: one greedy key per block (argmax_key)
    DecodeState* advance;      // kArgmax: when set, block 0 moves pos and step on by one
    const float* res;     // kResidual: the residual read (nullable: the stored row itself)
};

// Launch one batch-1 product: `blocks` blocks for each of the p.nseg segments
// (grid rows). `columns` in {384, 512, 1024, 1536, 2048}; returns
// hipErrorInvalidValue for an unsupported combination.
hipError_t launch_gemv(const GemvParams& p, int columns, int prologue, int epilogue, int form,
                       int rows_per_block, int blocks, hipStream_t stream);
int gemv_rows_per_block(int rows, int columns, int epilogue);

// The decode product with four waves splitting the columns (quantise prologue,
// residual epilogue with p.res, panel form); columns 2048.
hipError_t launch_gemv_splitk(const GemvParams& p, int columns, int rows, hipStream_t stream);

// ---- attention --------------------------------------------------------------
enum AttendMode { kAttendDecode = 0, kAttendPrefill = 1, kAttendRaw = 2 };

struct AttendParams {
    // kAttendDecode: q/k/v rows come from qkv [batch][3*d]; rotary is applied and
    //   k/v appended at pos[b]; grid (heads, batch).
    // kAttendPrefill: rotated q from q [count][d], positions first+t; grid (heads, count).
    // kAttendRaw: q [count][64], K/V [count][stride][64], lengths; grid (count).
    const float* qkv;
    const float* q;
    __half* kc;
    __half* vc;
    size_t seq_stride;    // elements between sequences' caches (decode batch)
    int layer, heads, capacity, d_model;
    const int32_t* pos;   // decode: [batch] positions (state->pos for batch 1)
    int pos_stride;       // int32 stride between positions (DecodeState vs plain array)
    int first;            // prefill: position of token 0
    const int32_t* lengths;
    int stride;           // raw: positions per problem
    const float* rope_cos;  // [max_positions][32]
    const float* rope_sin;
    float* out;
    int32_t* error;
};

hipError_t launch_attend(const AttendParams& p, int mode, int grid_x, int grid_y, int max_length,
                         hipStream_t stream);

// Causal attention of `count` prefill tokens at positions first.. (q [count][d]
// rotated, keys and values already appended): grid (heads, query tiles).
hipError_t launch_attend_prefill(const AttendParams& p, int heads, int count, hipStream_t stream);

// Batch-1 decode: norm + the q/k/v rows of each head + rotary + fp16 append +
// attention, one block per head (grid = heads, d_model = 64 heads).
// The fields a block needs at its start come first: they share the first 64 bytes
// of the argument segment, one scalar-cache line.
struct QkvAttendParams {
    const int8_t* W;      // fused q/k/v codes [3 d][d]
    const float* sW;      // [3 d][d/32]
    const float* x;       // residual stream [d] (kNorm)
    const float* gain;    // norm gains [d]
    __half* kc;           // this layer's cache [heads][capacity][64]
    __half* vc;
    DecodeState* state;   // token, pos, error flags
    int capacity;
    float eps;
    const int8_t* embW;   // kEmbedNorm: embedding codes/scales, token from state
    const float* embS;
    float embed_scale;
    int vocab;
    float* x_out;         // kEmbedNorm: block 0 writes the embedded row
    const float* rope_cos;
    const float* rope_sin;
    float* out;           // [d] attention output, head h at 64 h
    const unsigned long long* keys;  // kEmbedArgmax: the previous logits' block keys [nkeys]
    int nkeys;
    const float* logits;  // kEmbedArgmax: the previous logits (index 0 for the NaN rule)
    uint32_t* ids;        // kEmbedArgmax: block 0 writes ids[step - 1]
};
hipError_t launch_qkv_attend(const QkvAttendParams& p, int d_model, int prologue, int heads, hipStream_t stream);

// Rotary + fp16 append for `count` tokens of one sequence (prefill): writes the
// rotated queries to q_out [count][d] and keys/values into the cache.
hipError_t launch_rope_append(const float* qkv, float* q_out, __half* kc, __half* vc, int layer, int heads,
                              int capacity, int d_model, int first, int count, const float* rope_cos,
                              const float* rope_sin, hipStream_t stream);

// ---- multi-token products (i8 MFMA) ----------------------------------------------
// kGemmStoreSilu: y = silu(total); kGemmRope: the fused q/k/v rows of one
// layer, rotated and appended to the cache instead of stored (GemmParams::rope)
enum GemmEpilogue { kGemmStore = 0, kGemmResidual = 1, kGemmSilu = 2, kGemmStoreSilu = 3, kGemmRope = 4 };

// The q/k/v epilogue of a prefill product (kGemmRope): output columns are the q,
// k and v rows of `heads` heads of 64 (N == 3 * heads * 64); row m is position
// first + m. q is rotated into q_out [M][heads * 64], k rotated and v copied
// into this layer's fp16 caches [layers][heads][capacity][64]
// (crates/model/src/prefill.rs:10-99 with the rotary of ops.rs:131-141).
struct GemmRope {
    float* q_out;
    __half* kc;
    __half* vc;
    const float* cos;  // [positions][32]
    const float* sin;
    int layer, heads, capacity, first;
};

struct GemmParams {
    const int8_t* X;   // [M][K] quantised tokens
    const float* sx;   // [M] token scales
    const int8_t* W;   // [N][K]
    const float* sW;   // [N][K/32]
    int M, N, K;
    float* Y;          // [M][ldy] (kGemmSilu: [M][half])
    int ldy;
    int32_t* acc;      // dump only: [M][N][K/32]
    int half;          // kGemmSilu: gate rows 0..half-1, up rows half..2*half-1 (N == 2*half)
    // Optional float input rows [M][K] (nullable): the product quantises them
    // itself, after the zero-centred norm with `gain` when that is set
    // (ops.rs:44-58, 103-118). X and sx then receive the codes only where a
    // separate quantise launch is used (large grids); they must be valid.
    const float* Xf;
    const float* gain;
    float eps;
    GemmRope rope;     // kGemmRope only
};

hipError_t launch_gemm(const GemmParams& p, int epilogue, int form, bool dump, hipStream_t stream);
hipError_t launch_norm_quantise(const float* x, const float* gain, int count, int n, float eps, int8_t* codes,
                                float* scales, float* normed, hipStream_t stream);
// quantise_int8 of `count` rows of n floats that start x_stride floats apart
// (rows may overlap: the im2col rows of a strided convolution)
hipError_t launch_quantise_strided(const float* x, size_t x_stride, int count, int n, int8_t* codes, float* scales,
                                   hipStream_t stream);
hipError_t launch_embed_rows(const uint32_t* tokens, int count, const int8_t* E, const float* sE, int d, int vocab,
                             float scale, float* X, int32_t* error, hipStream_t stream);
// step_dev (nullable): the step is read from the device, so that a captured
// step graph writes each replay's ids in its own slot.
hipError_t launch_argmax_rows(const float* logits, int count, int n, uint32_t* tokens, uint32_t* ids, int steps,
                              int step, hipStream_t stream, const int32_t* step_dev = nullptr);
// pos[i] += by for each sequence; thread 0 also moves *step on (nullable).
hipError_t launch_advance_positions(int32_t* pos, int count, int by, hipStream_t stream, int32_t* step = nullptr);

// ---- speech path (rn_whistle.hip) ---------------------------------------------
// The stem's first convolution (kernel 3, stride 1, pad 1) + silu into h1 [F][d].
hipError_t launch_stem(const float* mel, const float* conv1, int F, int M, int d, float* h1, hipStream_t stream);

struct HeadSection {
    int col;             // first column of the section in a source row
    const float* gain;   // head norm gains [64], or null
    int rotary;          // rotate at position pos0 + frame
    float scale_mul;     // multiplies the stored scale
    int8_t* codes;       // [frames][heads][64]
    float* scales;       // [frames][heads]
};
struct HeadCodesParams {
    const float* src;    // [frames][src_stride]
    int src_stride, frames, heads, nsec;
    HeadSection sec[3];
    const float* rope_cos;  // [positions][32]
    const float* rope_sin;
    int pos0;
    float eps;
};
hipError_t launch_head_codes(const HeadCodesParams& p, hipStream_t stream);

struct Int8AttendParams {
    const int8_t* qc;    // [queries][heads][64]
    const float* qs;     // [queries][heads] (times 1/sqrt(64))
    const int8_t* kc;    // [frames][heads][64]
    const float* ks;     // [frames][heads]
    const int8_t* vc;
    const float* vs;
    int frames, heads;
    float* out;          // [queries][out_stride], head h at column 64 h
    int out_stride;
};
hipError_t launch_int8_attend(const Int8AttendParams& p, int queries, hipStream_t stream);

// The decoder's cross-attention for one token (cross.rs:126-170 up to the
// attention output): zero-centred norm of x with the cross gains, the head's
// 64 rows of the cross q product, per-head q norm and int8 codes, int8 scores
// over the layer's memory, softmax, and the value sums of the 32 position
// classes, written per class (part[c][64 h + i]); a kClassSum product adds them.
struct CrossAttendParams {
    const int8_t* W;     // cross q codes [d][d]
    const float* sW;     // [d][d/32]
    const float* x;      // residual stream [d]
    const float* gain;   // norm_cross [d]
    const float* q_gain; // q_norm [64]
    float eps;
    const int8_t* kc;    // layer memory [frames][heads][64] and scales [frames][heads]
    const float* ks;
    const int8_t* vc;
    const float* vs;
    int frames, heads;
    float* part;         // [32][d]
};
hipError_t launch_cross_attend(const CrossAttendParams& p, int d_model, hipStream_t stream);

// A codebook-quantised matrix on the device: the archive blob as stored
// (packed indices [rows][row_bytes], then fp16 norms [rows][padded/group]; the
// allocation runs at least 16 KB past the norms) and the host-derived tables.
struct CodebookParams {
    const uint8_t* packed;
    const uint16_t* norms;
    int rows, columns, padded, group, bits;  // bits 5: ternary crumbs
    int row_bytes;                           // padded * index_bits / 8
    int cpr;                                 // 16-byte chunks per row
    float inv_cpr;                           // 1 / cpr
    int rows_per_block;                      // rows of a wave's row group (set by the launcher)
    int iters;                               // row groups per block (set by the launcher)
    uint32_t lut[4];                         // IntegerLevels table, 16 int8
    float lscale;                            // IntegerLevels scale
    float levels[16];                        // float levels (dequantise_row)
    float wht_scale;                         // 1 / sqrt(group)
};
// rotated [count][padded] inputs -> y [count][rows] (acc nullable: [count][rows][groups])
hipError_t launch_codebook_product(const CodebookParams& p, const float* x, int count, float* y, int32_t* acc,
                                   hipStream_t stream);
// up to kCodebookJobs products of one vector each, in one launch: the matrices
// share rows, padded width, bits and group (the integer path)
constexpr int kCodebookJobs = 4;
struct CodebookJob {
    CodebookParams p;
    const float* x;  // rotated [padded]
    float* y;        // [rows]
};
struct CodebookJobs {
    CodebookJob job[kCodebookJobs];
};
hipError_t launch_codebook_product_jobs(const CodebookJobs& jobs, int n, hipStream_t stream);
// The float products of any width (1-5): fill_rows_float (batch false, one
// result per token and row in the vector order) or multiply_batch's float tile
// (batch true); rotated [count][padded] -> y [count][rows].
hipError_t launch_codebook_float(const CodebookParams& p, const float* x, int count, float* y, bool batch,
                                 hipStream_t stream);
hipError_t launch_codebook_rotate(const float* x, int count, int columns, int padded, int group, float scale,
                                  float* rotated, hipStream_t stream);
hipError_t launch_codebook_dequantise(const CodebookParams& p, int row, float* out, hipStream_t stream);

// The multi-lane hyper-connection (lanes.rs): route after the three products.
constexpr int kMaxLanes = 16;
struct LanesRouteParams {
    int lanes, width, layer, slot;
    const float* a_pre;    // [layers]
    const float* a_post;
    const float* a_res;
    const float* b_pre;    // [layers][lanes]
    const float* b_post;
    const float* b_res;    // [layers][lanes][lanes]
    const float* stream;   // [lanes][width]
    const float* pre;      // [lanes] the phi_pre rows of this layer
    float* post;           // [lanes] in: the phi_post rows; out: the post gains
    float* residual;       // [lanes][lanes] in: the phi_res rows; out: the Sinkhorn mix
    float* input;          // [width]
};
hipError_t launch_lanes_prologue(const float* stream, int n, float* out, hipStream_t s);
hipError_t launch_lanes_route(const LanesRouteParams& p, hipStream_t s);
hipError_t launch_lanes_combine(int lanes, int width, const float* post, const float* residual, const float* stream,
                                const float* delta, float* next, hipStream_t s);

// kronecker_apply for 32 x 32 factors over `count` inputs [count][1024].
hipError_t launch_kronecker32(const float* input, const float* left, const float* right, int count, float* output,
                              hipStream_t stream);

// One int8 row dequantised: out[k] = codes[k] * scales[k / group].
hipError_t launch_dequantise_i8(const int8_t* codes, const float* scales, int columns, int group, float* out,
                                hipStream_t stream);

// The speech front end (frontend.rs): device tables built on the host.
struct FrontendParams {
    int mels, fft_size, log2_size, window, hop;
    const float* window_gain;  // [window] Hann gains
    const float* twiddle_cos;  // [fft_size / 2]
    const float* twiddle_sin;
    const float* mel_weights;  // [fft_size / 2 + 1][mels]
};
// samples [n] -> data [n / hop + 1][mels] normalised; spread[0] the spread,
// spread[1 .. mels] scratch for the per-mel deviations
hipError_t launch_log_mel(const FrontendParams& p, const float* samples, int n, float* data, float* spread,
                          hipStream_t stream);

// The grammar-constrained choice (generator.rs:99-117): the chosen token (or
// the given one), whether an allowed token existed, and allowed_statistics.
struct Choice {
    uint32_t token;
    int32_t constrained;
    float probability;
    float mass;
};
hipError_t launch_constrained_choice(const float* logits, const uint8_t* allowed, int n, int token, Choice* out,
                                     hipStream_t stream);
hipError_t launch_add(const float* a, const float* b, size_t n, float* out, hipStream_t stream);

// ---- elementwise / helpers ----------------------------------------------------
hipError_t launch_quantise_rows(const float* x, int count, int columns, int8_t* codes, float* scales,
                                hipStream_t stream);
hipError_t launch_norm_rows(const float* x, const float* gain, int count, int n, float eps, float* out,
                            hipStream_t stream);
hipError_t launch_fast_exp(const float* x, float* y, int n, int op, hipStream_t stream);  // op 0..3: fast_exp, silu, expf, sigmoid
hipError_t launch_finish_push(const float* x, const float* gain, int n, float eps, float* hidden,
                              DecodeState* state, hipStream_t stream);
// Second stage of the greedy argmax: reduces the per-block keys of the logits
// product, writes the token into the state and ids[step], advances step and pos.
// mode 0: token = the keys' choice; ids[step] = token; step and pos move on.
// mode 1 (after a greedy run whose steps moved pos and step themselves): the
// last step's choice into ids[step - 1], nothing moved.
hipError_t launch_argmax_finalize(const unsigned long long* keys, int nkeys, const float* logits,
                                  DecodeState* state, uint32_t* ids, hipStream_t stream, int mode = 0);
// The start of a greedy run with the choice folded into the next step's first
// kernel: the state (token, pos, step 0, ids capacity), every block key set to
// the key of `token` and logits[0] to 0, so that step 0 chooses `token`.
hipError_t launch_greedy_start(DecodeState* state, uint32_t token, int32_t pos, uint32_t ids_capacity,
                               unsigned long long* keys, int nkeys, float* logits, hipStream_t stream);
// Overwrites token/pos/step/ids_capacity.
hipError_t launch_set_state(DecodeState* state, uint32_t token, int32_t pos, uint32_t step, uint32_t ids_capacity,
                            hipStream_t stream);

}  // namespace rn
