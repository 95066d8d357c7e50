/*
 * rustyneedle.h — C ABI of the MI355X (gfx950) Needle token loop.
 *
 * The library replaces the CPU hot path of rustyneedle behind its own seams:
 *   - the kernels API (QuantisedMatrix and the free functions re-exported at
 *     crates/kernels/src/lib.rs:17-25),
 *   - the model API (Model / Session, crates/model/src/session.rs:17-177),
 *   - the greedy loop that the Engine trait drives
 *     (crates/generate/src/generator.rs:199-265, crates/needle/src/engine.rs:14-18).
 * Reference citations below are file:line in mcnairstudios/rustyneedle.
 *
 * Conventions
 *   - Every entry point returns an int status: RN_OK (0) or a negative RN_ERR_*.
 *     rn_last_error() returns the calling thread's last message. No C++
 *     exception crosses the ABI. The reference panics on shape mismatches
 *     (matrix.rs:156-157, neon.rs:44); here they are RN_ERR_ARGUMENT.
 *   - Handles are opaque and freed by the caller. Device pointers passed to the
 *     kernels API are caller-owned device memory (rn_malloc); `stream` is a
 *     hipStream_t passed as void* (NULL = the default stream).
 *   - Model / session entry points take host pointers for their inputs and
 *     outputs and keep weights, caches and scratch resident in device memory.
 *   - Numerics: int8 weight codes with one fp32 scale per `group` columns;
 *     activations are quantised per row with an absmax scale (ops.rs:103-118);
 *     the per-row product epilogue is sequential over groups, in the panel form
 *     fmaf((float)acc, sW*sx, total) (panel.rs:184-188) for layer matrices and
 *     the plane form total + ((float)acc*sW)*sx (neon.rs:180) for the tied
 *     embedding. Integer accumulators and greedy token ids match the CPU
 *     restatement bit for bit.
 */
#ifndef RUSTYNEEDLE_H
#define RUSTYNEEDLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RN_ABI_VERSION 1

enum {
    RN_OK = 0,
    RN_ERR_ARGUMENT = -1, /* bad shape, null pointer, unsupported geometry */
    RN_ERR_DEVICE = -2,   /* a HIP call failed (no device, launch failure, ...) */
    RN_ERR_CAPACITY = -3, /* a session would grow past its KV capacity */
    RN_ERR_STATE = -4,    /* call out of order (e.g. logits before any push) */
    RN_ERR_MEMORY = -5    /* device or host allocation failed */
};

/* Product epilogue form of a matrix (see the header comment). */
enum { RN_FORM_PANEL = 0, RN_FORM_PLANE = 1 };

const char* rn_last_error(void);
int rn_abi_version(void);

/* ---- device plumbing (no reference counterpart: the reference is host-only) ---- */
int rn_device_count(int* count);
int rn_device_set(int device);
int rn_malloc(void** ptr, size_t bytes);
int rn_free(void* ptr);
int rn_memcpy_htod(void* dst, const void* src, size_t bytes);
int rn_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int rn_memcpy_dtod(void* dst, const void* src, size_t bytes);
int rn_stream_create(void** stream);
int rn_stream_destroy(void* stream);
int rn_stream_synchronize(void* stream);
int rn_event_create(void** event);
int rn_event_destroy(void* event);
int rn_event_record(void* event, void* stream);
int rn_event_elapsed_ms(void* start, void* stop, float* ms);

/* ---- kernels API: QuantisedMatrix (crates/kernels/src/matrix.rs:19-441) -------- */
typedef struct rn_matrix rn_matrix;

/* Replaces QuantisedMatrix::from_archive/from_parts (matrix.rs:35-59): host codes
 * [rows][columns] int8 and scales [rows][columns/group] f32 are copied to the
 * device. columns must be 384, 512, 1024, 1536 or 2048; group must be 32. */
int rn_matrix_create_i8(const int8_t* codes, const float* scales, int rows, int columns, int group,
                        int form, rn_matrix** out);
int rn_matrix_free(rn_matrix* m);
/* QuantisedMatrix::rows/columns/group (matrix.rs:61-75). */
int rn_matrix_shape(const rn_matrix* m, int* rows, int* columns, int* group);

/* QuantisedMatrix::multiply_vector (matrix.rs:155-165) with the activation
 * quantisation of plane_input (matrix.rs:205-214) done on the device:
 * y[rows] = W . quantise_int8(x[columns]). acc (nullable) receives the int32
 * accumulator of every (row, group): [rows][columns/group]. Device pointers. */
int rn_matrix_multiply_vector(const rn_matrix* m, const float* x, float* y, int32_t* acc, void* stream);
/* The same product (int8 matrices of 384 or 512 columns) with the kernel
 * instance of `rows_per_block` output rows a block (8, 16 or 32) instead of the
 * one rn_matrix_multiply_vector picks from the shape; the results are the same.
 * For measurement: the instance a 2048-row product runs (8) over a tall matrix. */
int rn_matrix_multiply_vector_rows(const rn_matrix* m, const float* x, float* y, int rows_per_block, void* stream);

/* QuantisedMatrix::multiply_fused (matrix.rs:167-193): one launch over `count`
 * (<= 8) matrices of equal columns/group/form that share the input x. */
int rn_matrix_multiply_fused(const rn_matrix* const* ms, int count, const float* x, float* const* ys,
                             void* stream);

/* QuantisedMatrix::multiply_batch (matrix.rs:330-389): x [count][columns],
 * y [count][rows] token-major (matrix.rs:384-388). acc nullable:
 * [count][rows][columns/group]. Runs on i8 MFMA. */
int rn_matrix_multiply_batch(const rn_matrix* m, const float* x, int count, float* y, int32_t* acc,
                             void* stream);

/* rn_matrix_multiply_batch without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The input rows' int8 codes and scales go to a fixed scratch array that the
 * library holds on each GPU until the process ends (4 MiB of codes + 4096
 * scales): count <= 4096 and count * columns rounded up to 256 <= 4 MiB, or
 * RN_ERR_ARGUMENT. Every call on one GPU shares that GPU's array, which keeps
 * the last call's contents. Calls outside stream capture are ordered on the
 * device: each call's stream waits for the previous call's kernels (an event
 * per GPU, recorded under a lock), so calls from several threads or streams
 * run one after another. Under stream capture no such wait is recorded: the
 * graphs captured from this call must not run concurrently with each other or
 * with other calls on the same GPU. Codebook matrices need no scratch and run
 * as rn_matrix_multiply_batch. Device pointers, as rn_matrix_multiply_batch. */
int rn_matrix_multiply_batch_noalloc(const rn_matrix* m, const float* x, int count, float* y, int32_t* acc,
                                     void* stream);

/* Host-slice forms, with the reference's signatures: the input slice is host
 * memory, the output slice host memory the call fills before it returns.
 * Each copies the input to a staging buffer the matrix owns, runs the device
 * entry point above on the matrix's own stream, copies the output back and
 * synchronises; calls on one matrix from several threads are serialised
 * (QuantisedMatrix is Send + Sync). The staging buffer is allocated on the
 * first call and grown as needed.
 *   QuantisedMatrix::multiply_vector(&self, rotated: &[f32], output: &mut [f32])
 *     (matrix.rs:155-165): x [padded columns], y [rows].
 *   QuantisedMatrix::multiply_batch(&self, rotated: &[f32], count, output: &mut [f32])
 *     (matrix.rs:330-389): x [count][padded columns], y [count][rows].
 *   QuantisedMatrix::prepare_batch (matrix.rs:123-138), codebook matrices:
 *     x [count][columns] -> rotated [count][padded columns].
 * For int8 matrices the padded columns are the columns. */
int rn_matrix_multiply_vector_host(const rn_matrix* m, const float* x, float* y);
int rn_matrix_multiply_batch_host(const rn_matrix* m, const float* x, int count, float* y);
int rn_matrix_prepare_host(const rn_matrix* m, const float* x, int count, float* rotated);

/* QuantisedMatrix::dequantise_row (matrix.rs:140-153) for int8 codes: out[k] =
 * code * scale(group of k); for codebook matrices (level[index] * norm) then
 * the Walsh-Hadamard transform of each group, on the device. Host output of
 * `columns` floats. */
int rn_matrix_dequantise_row(const rn_matrix* m, int row, float* out);

/* ---- the codebook weight format (docs/format.md "Codebook-quantised matrices") ----
 * Replaces QuantisedMatrix::from_archive/from_parts (matrix.rs:35-59) for a
 * kind-3 record (cact record.rs:7-84): `blob` is the record's bytes as the
 * archive holds them (packed indices LSB first, rows x padded x index_bits / 8
 * bytes, then rows x padded / group fp16 norms), `codebook` the archive's 28
 * levels (2-bit 0..3, 3-bit 4..11, 4-bit 12..27). bits 1..4 or 5 (ternary
 * crumbs); group 64, 128 or 256. The blob is copied to the device as is.
 * The multiply entry points above then take the ROTATED input of
 * rn_matrix_prepare ([count][padded] floats), quantise it per group and run
 * the integer path: 2-bit matrices the panel form (panel.rs:153-197), 4-bit and
 * ternary ones the plane form (neon.rs:126-183). multiply_fused on codebook
 * matrices launches once per matrix. 1- and 3-bit matrices have no integer
 * levels in the reference (matrix.rs:559-563): their products are the float
 * path below (no acc). */
int rn_matrix_create_codebook(const uint8_t* blob, size_t blob_bytes, int rows, int columns, int group, int bits,
                              const float* codebook, int codebook_len, rn_matrix** out);
/* The float path of a codebook matrix, the one the reference takes on x86-64
 * for every width (docs/portability.md:10) and everywhere for 1- and 3-bit
 * ones. Rotated inputs (not quantised), device pointers.
 *   vector: fill_rows_float (matrix.rs:427-440) with LookupTable::dot_group
 *     (matrix.rs:610-620): per group, each of the 8 / index_bits lanes of a
 *     byte sums level * input over the group's bytes in order, the lanes are
 *     summed in order (3-bit: one sum over the positions), then
 *     total += partial * norm over the groups in order.
 *   batch: multiply_batch's float tile (matrix.rs:356-378): the row expanded
 *     as level * norm (matrix.rs:390-399) and dotted with each input in
 *     eight lanes (matrix.rs:488-497). */
int rn_matrix_multiply_vector_float(const rn_matrix* m, const float* rotated, float* y, void* stream);
int rn_matrix_multiply_batch_float(const rn_matrix* m, const float* rotated, int count, float* y, void* stream);
/* QuantisedMatrix::padded_columns (matrix.rs:69-71); columns for int8 matrices. */
int rn_matrix_padded_columns(const rn_matrix* m, int* padded);
/* QuantisedMatrix::prepare / prepare_batch (matrix.rs:123-138): x [count][columns]
 * -> rotated [count][padded], zero-padded and rotated group by group
 * (walsh.rs:41-80). Codebook matrices only. Device pointers. */
int rn_matrix_prepare(const rn_matrix* m, const float* x, int count, float* rotated, void* stream);

/* ---- the .cact archive (crates/cact; docs/format.md) ---------------------------
 * A memory-mapped, little-endian archive: 196-byte header, codebook levels, a
 * directory of 44-byte tensor records, 64-byte aligned blobs. Host-side; the
 * pointers returned stay valid until rn_archive_close. */
typedef struct rn_archive rn_archive;
/* Geometry (geometry.rs:10-37): the header fields in file order; global_layers
 * joins global_mask_lo/hi; only the first engram_order_count orders and
 * engram_site_count sites are meaningful. */
typedef struct {
    uint32_t tensor_count, codebook_len, kv_window, kv_bits, vocab, out_vocab, d_model, num_heads, num_kv_heads,
        num_layers, qk_head_dim, v_head_dim, max_seq_len, hada_n, mhc_lanes, sliding_window;
    uint64_t global_layers;
    uint32_t qkv_conv_taps, engram_slots, engram_sub_dim, engram_tables, engram_conv_taps, engram_conv_dilation,
        engram_seed_heads, engram_order_count, engram_orders[4], engram_site_count, engram_sites[16];
    float rope_theta;
} rn_geometry;
/* ElementKind (record.rs:7-25) */
enum { RN_KIND_HALF = 1, RN_KIND_SINGLE = 2, RN_KIND_CODEBOOK = 3, RN_KIND_RAW = 4 };
/* TensorRecord (record.rs:27-51): shape[rank..4) is 0; bits 5 marks ternary crumbs. */
typedef struct {
    int kind, rank;
    uint32_t shape[4];
    uint64_t offset, nbytes;
    uint32_t group_size, bits;
} rn_tensor_record;
/* Archive::open (archive.rs:37-41) with the checks of Archive::from_map
 * (archive.rs:43-70): format tag, truncation, element kinds, every tensor inside
 * the file and aligned to its element width. Errors carry the reference's
 * messages (error.rs:15-26). */
int rn_archive_open(const char* path, rn_archive** out);
/* The same over bytes in memory (copied). */
int rn_archive_from_memory(const uint8_t* bytes, size_t nbytes, rn_archive** out);
int rn_archive_close(rn_archive* archive);
int rn_archive_geometry(const rn_archive* archive, rn_geometry* out);     /* Archive::geometry (archive.rs:72-74) */
int rn_archive_codebook(const rn_archive* archive, const float** values, int* count); /* archive.rs:76-78 */
int rn_archive_record(const rn_archive* archive, int index, rn_tensor_record* out);  /* archive.rs:80-82 */
int rn_archive_tensor_bytes(const rn_archive* archive, int index, const uint8_t** data, size_t* nbytes); /* archive.rs:88-91 */
/* QuantisedMatrix::from_archive (matrix.rs:35-40): a kind-3 record to the device
 * (rn_matrix_create_codebook with the record's shape, group and bits). */
int rn_matrix_from_archive(const rn_archive* archive, int index, rn_matrix** out);

/* ---- the multi-lane hyper-connection (crates/model/src/lanes.rs) ----------------
 * LaneWeights::load (lanes.rs:31-45): the lane tensors a_pre/a_post/a_res
 * [layers], b_pre/b_post [layers][lanes], b_res [layers][lanes][lanes] (host
 * floats, copied) and the three codebook routing matrices (kept by reference:
 * phi_pre and phi_post of layers x lanes rows, phi_res of layers x lanes^2
 * rows, all over the lanes x width stream). lanes <= 16. An rn_lanes holds
 * the scratch of its route (normalised and rotated stream, pre gains): calls
 * on one rn_lanes must not overlap. */
typedef struct rn_lanes rn_lanes;
int rn_lanes_create(int lanes, int width, int layers, const float* a_pre, const float* a_post, const float* a_res,
                    const float* b_pre, const float* b_post, const float* b_res, const rn_matrix* phi_pre,
                    const rn_matrix* phi_post, const rn_matrix* phi_res, rn_lanes** out);
int rn_lanes_free(rn_lanes* lanes);
/* LaneWeights::route (lanes.rs:48-84) on device pointers: stream [lanes][width]
 * -> input [width], post [lanes], residual [lanes][lanes], bit for bit:
 * unit_rms, fake_quantise_int8, prepare and the products in the reference's
 * order, the gates (sigmoid) and sinkhorn_in_place over the device restatement
 * of the C library's expf (rn_libm_exp). */
int rn_lanes_route(rn_lanes* lanes, int layer, int slot, const float* stream, float* input, float* post,
                   float* residual, void* stream_handle);
/* LaneWeights::combine_into (lanes.rs:86-98): next [lanes][width]. */
int rn_lanes_combine(const rn_lanes* lanes, const float* post, const float* residual, const float* stream,
                     const float* block_delta, float* next, void* stream_handle);

/* ---- Needle 3 (crates/model/src) --------------------------------------------------
 * Model::from_archive + with_depth (model.rs:50-78) over an open archive: the
 * canonical tensor order (layout.rs:176-257) with the probe heads and no audio
 * encoder; every codebook matrix and float tensor goes to the device (the
 * archive may be closed afterwards). depth <= 0 keeps every layer; otherwise
 * ladder::select (RN_ERR_ARGUMENT where it returns None). Head dimensions of
 * 64, a Hadamard size of 1024 (32 x 32 factors), d_model <= 1024. */
typedef struct rn_n3_model rn_n3_model;
typedef struct rn_n3_session rn_n3_session;
int rn_n3_model_open(const rn_archive* archive, int depth, rn_n3_model** out);
int rn_n3_model_free(rn_n3_model* model);
int rn_n3_model_active_layers(const rn_n3_model* model, int* layers, int* count); /* Model::active_layers */
int rn_n3_model_output_vocab(const rn_n3_model* model, int* count);               /* geometry.rs:117-123 */
/* Session::new (session.rs:30-42) with room for `capacity` tokens (<= 8192). */
int rn_n3_session_create(const rn_n3_model* model, int capacity, rn_n3_session** out);
int rn_n3_session_free(rn_n3_session* session);
/* Session::push (session.rs:76-148) and Session::feed (session.rs:58-74; at
 * least 4 tokens run as batched prefills, prefill.rs:10-99, of up to 256 tokens,
 * with each token's arithmetic a push's). Tokens below the vocabulary;
 * RN_ERR_ARGUMENT past the capacity. */
int rn_n3_session_push(rn_n3_session* session, uint32_t token);
int rn_n3_session_feed(rn_n3_session* session, const uint32_t* tokens, int count);
/* Generator::run_turn's greedy loop (generator.rs:199-230, argmax at 257-265)
 * without grammar: token = first; `steps` times { push(token); logits; token =
 * argmax over output_vocab; ids[i] = token } (host ids). The argmax stays on
 * the device and feeds the next push. */
int rn_n3_session_decode_greedy(rn_n3_session* session, uint32_t first, int steps, uint32_t* ids);
/* #[derive(Clone)] on Session (session.rs:17): a new session holding a copy of
 * the whole state, which then continues independently. Generator::new keeps a
 * base session with the system prompt and clones it per turn and on reset
 * (generator.rs:41-46). */
int rn_n3_session_clone(const rn_n3_session* session, rn_n3_session** out);
/* The token loop of Generator::run_turn (generator.rs:99-130) while no grammar
 * is active: while n < max_tokens && len + 1 < window { next = argmax(logits)
 * (generator.rs:157-165); ids[n++] = next; push(next); a token of stops
 * (im_end, eos) ends the loop after its push }. run_turn counts the think_start
 * token it fed in `generated`, so its max_new_tokens is max_tokens + 1 here.
 * window <= 0 takes the archive's max_seq_len. *count = n; *finished = 1 when a
 * stop token ended the loop. The argmax feeds the push on the device; the host
 * reads each token (for the stop test) while the push of it runs. Needs a
 * pushed token; RN_ERR_ARGUMENT when the loop could pass the capacity. */
int rn_n3_session_run_turn(rn_n3_session* session, int max_tokens, int window, const uint32_t* stops, int stop_count,
                           uint32_t* ids, int* count, int* finished);
/* generator.rs:104-116 while a tool-call grammar is active: the session's
 * logits, argmax_allowed over `allowed` (output_vocab host bytes, non-zero =
 * allowed; the grammar's TokenBytes::allowed), the argmax where nothing is
 * allowed, and allowed_statistics of the choice (rn_choice below, host). The
 * caller pushes out->token with rn_n3_session_push. */
typedef struct rn_choice rn_choice;
int rn_n3_session_choose_allowed(rn_n3_session* session, const uint8_t* allowed, rn_choice* out);
int rn_n3_session_length(const rn_n3_session* session, int* length);
/* Session::logits (session.rs:151-165): output_vocab floats (host). */
int rn_n3_session_logits(rn_n3_session* session, float* logits);
/* The final hidden state [d_model] and Session::cells [active + 1][d_model] (host). */
int rn_n3_session_hidden(rn_n3_session* session, float* hidden);
int rn_n3_session_cells(rn_n3_session* session, float* cells);
/* Session::head_output / pooled_readout (session.rs:125-135): the head with
 * `code`; *count is 0 when there is none (the reference's None). Host output
 * of `capacity` floats. */
int rn_n3_session_head_output(rn_n3_session* session, int code, float* out, int capacity, int* count);
int rn_n3_session_pooled_readout(rn_n3_session* session, int code, float* out, int capacity, int* count);
/* The int8 cache of a layer (attention.rs:36-44): keys / values [length][kv][64],
 * scales [kv][length] (host). RN_ERR_ARGUMENT for a layer outside the active
 * ladder selection (whose cache the reference never fills). */
int rn_n3_session_cache(rn_n3_session* session, int layer, int8_t* keys, float* key_scales, int8_t* values,
                        float* value_scales);
int rn_n3_session_stream(const rn_n3_session* session, void** stream);

/* ---- the depth ladder (crates/model/src/ladder.rs) -------------------------------
 * ladder::order (ladder.rs:1-20): the order in which layers join as depth grows
 * (host). ladder::select (ladder.rs:22-29): the sorted first `depth` of them;
 * RN_ERR_ARGUMENT where the reference returns None (depth outside
 * [min(2, layers), layers]). */
int rn_ladder_order(int layers, int32_t* order);
int rn_ladder_select(int layers, int depth, int32_t* chosen);

/* ops::kronecker_apply (ops.rs:166-217), the factor product of the Hadamard MLP
 * (hadamard.rs:100-106): out = L^T . X . R for each of `count` inputs X
 * [32][32] (device pointers, [count][1024] in and out; L and R [32][32]). Only
 * 32 x 32 factors: those the reference runs on its aarch64 path
 * (ops.rs:220-297), whose fused multiply-adds in index order this follows. */
int rn_kronecker_apply(const float* input, const float* left, int left_size, const float* right, int right_size,
                       int count, float* output, void* stream);

/* ops::quantise_int8 (ops.rs:112-118) for `count` rows of `columns` floats on
 * the device: codes [count][columns], scales [count]. */
int rn_quantise_int8(const float* x, int count, int columns, int8_t* codes, float* scales, void* stream);

/* ops::fast_exp (ops.rs:82-90) and ops::silu (ops.rs:73-76) applied elementwise
 * on the device (exposed for parity checks of the transcendental semantics). */
int rn_fast_exp(const float* x, float* y, int n, void* stream);
int rn_silu(const float* x, float* y, int n, void* stream);

/* f32::exp as the reference calls it (the C library's expf: ops::sigmoid,
 * ops.rs:68-71, sinkhorn_in_place, ops.rs:198-217, ProbeHead::observe,
 * heads.rs:138-150) and ops::sigmoid over it, elementwise on the device; equal
 * bit for bit to glibc's x86-64 expf. Exposed for parity checks. */
int rn_libm_exp(const float* x, float* y, int n, void* stream);
int rn_sigmoid(const float* x, float* y, int n, void* stream);
/* f32::ln as the reference calls it (the C library's logf: the log-mel
 * features, frontend.rs:96-99), elementwise on the device; equal bit for bit to
 * this image's glibc logf on all 2^32 inputs. Exposed for parity checks. */
int rn_libm_log(const float* x, float* y, int n, void* stream);
/* The division-free reciprocal the fused Needle 3 step uses for the Sinkhorn
 * normalisation (1.0f / total, ops.rs:198-217): v_rcp_f32 and one Newton step,
 * elementwise on the device; equal to the IEEE division for every x in
 * [2^-126, 2^126), the only inputs it is given. Exposed for that check. */
int rn_reciprocal(const float* x, float* y, int n, void* stream);

/* ops::zero_centred_norm (ops.rs:44-50) for `count` rows of `n` floats on the
 * device (n a multiple of 8, <= 4096). */
int rn_zero_centred_norm(const float* x, const float* gain, int count, int n, float* out, void* stream);

/* kernels::attend_head (kernels/src/attention.rs:251-280) over an fp16 cache for
 * `count` independent (query, cache) problems: q [count][head_dim] f32 (already
 * rotated), K/V [count][stride][head_dim] fp16 bits, lengths [count] int32 (<=
 * stride), out [count][head_dim]. head_dim must be 64. Device pointers. */
int rn_attend_heads(const float* q, const uint16_t* K, const uint16_t* V, const int32_t* lengths,
                    int count, int stride, int head_dim, float* out, void* stream);

/* ---- model API: Model / Session (crates/model/src/model.rs, session.rs) -------- */
typedef struct {
    int layers, d_model, heads, head_dim, ffn, vocab, group, max_positions;
    float rope_theta, norm_eps;
} rn_config;

typedef struct { const int8_t* codes; const float* scales; } rn_qmat_host;

typedef struct {
    rn_qmat_host qkv;     /* [3*d][d]: rows q (heads*head_dim), then k, then v */
    rn_qmat_host out;     /* [d][d] */
    rn_qmat_host gate_up; /* [2*ffn][d]: gate rows 0..ffn-1, up rows ffn..2*ffn-1 */
    rn_qmat_host down;    /* [d][ffn] */
    const float* norm_attn; /* [d] zero-centred gains */
    const float* norm_ffn;  /* [d] */
} rn_layer_host;

typedef struct {
    rn_qmat_host embedding;  /* [vocab][d], tied with the logits product */
    const float* norm_final; /* [d] */
    const rn_layer_host* layers;
} rn_weights_host;

typedef struct rn_model rn_model;
typedef struct rn_session rn_session;
typedef struct rn_batch rn_batch;

/* Model::open / Model::build (model.rs:51-74): uploads all weights and the
 * rotary table (ops.rs:127-141, tabulated for max_positions). Supported
 * geometry: d_model 512, head_dim 64, heads*head_dim == d_model, ffn 2048,
 * group 32, vocab a multiple of 64. */
int rn_model_create(const rn_config* config, const rn_weights_host* weights, rn_model** out);
/* The same model built from the seeded synthetic generators (rn_synth_*) with
 * the tensor names listed at rn_synth_tensor_name. */
int rn_model_create_synthetic(const rn_config* config, uint64_t seed, rn_model** out);
int rn_model_free(rn_model* model);
int rn_model_config(const rn_model* model, rn_config* out);
/* The tabulated rotary cos/sin, [max_positions][head_dim/2] each (host out). */
int rn_model_rotary_table(const rn_model* model, float* cos_out, float* sin_out);

/* Session::new (session.rs:30-42) with a device KV cache of `capacity` positions
 * per layer and head (fp16, [layers][heads][capacity][head_dim]). */
int rn_session_create(const rn_model* model, int capacity, rn_session** out);
int rn_session_free(rn_session* session);
/* Session: Clone (session.rs:17; generator.rs:45) — a device-to-device copy. */
int rn_session_clone(const rn_session* session, rn_session** out);
/* Session::len (session.rs:44-46). */
int rn_session_len(const rn_session* session, int* length);
/* Keep only the first `length` (<= len) cached positions. No reference
 * counterpart: the reference returns to a prefix by cloning a base session
 * (generator.rs:45); this does it in place without a device allocation. The
 * hidden state is cleared until the next push or feed. */
int rn_session_truncate(rn_session* session, int length);
/* Replace the cache contents with `length` positions (host fp16 bits,
 * [layers][heads][length][head_dim]); used to pre-fill a context. */
int rn_session_set_cache(rn_session* session, int length, const uint16_t* keys, const uint16_t* values);
/* Read the first `length` cached positions back (same layout). */
int rn_session_get_cache(const rn_session* session, int length, uint16_t* keys, uint16_t* values);
/* Session::push (session.rs:72-148). */
int rn_session_push(rn_session* session, uint32_t token);
/* Session::feed (session.rs:56-70): batched prefill on i8 MFMA products. */
int rn_session_feed(rn_session* session, const uint32_t* tokens, int count);
/* The final-norm hidden state after the last push/feed (host out, d_model). */
int rn_session_hidden(const rn_session* session, float* out);
/* Session::logits (session.rs:166-177) (host out, vocab floats). */
int rn_session_logits(rn_session* session, float* out);
/* Generator::run_turn's greedy loop (generator.rs:199-230, argmax at 257-265)
 * without grammar: token = first; `steps` times { push(token); logits;
 * token = argmax; ids[i] = token }. Each step is one replay of a captured
 * hipGraph; the argmax stays on the device and feeds the next embedding. */
int rn_session_decode_greedy(rn_session* session, uint32_t first, int steps, uint32_t* ids);

/* ---- grammar-constrained choice (generator.rs:99-117, 147-194) ----------------
 * While a tool-call grammar is active the generator picks
 * argmax_allowed(logits, allowed) (the first allowed index of the largest
 * allowed value; a NaN wins only as the first allowed value), falls back to
 * argmax when nothing is allowed, and accumulates allowed_statistics of the
 * choice: probability = fast_exp(l[t] - peak_allowed) / total_allowed and
 * mass = total_allowed * fast_exp(peak_allowed - peak_all) / total_all, the
 * totals summed sequentially in index order as the reference does. */
struct rn_choice {
    uint32_t token;      /* the choice (or the token asked for) */
    int32_t constrained; /* 1: argmax_allowed found a token; 0: nothing allowed, argmax */
    float probability;
    float mass;
};
/* logits [n] f32, allowed [n] bytes (non-zero = allowed) and out are device
 * pointers; token < 0 chooses, token >= 0 gives the statistics of that token. */
int rn_choose_allowed(const float* logits, const uint8_t* allowed, int n, int token, rn_choice* out, void* stream);
/* The session's logits (as rn_session_logits, left on the device) and the
 * constrained choice over them: allowed is a host mask of vocab bytes (the
 * grammar's TokenBytes::allowed, generator.rs:104), out a host rn_choice. */
int rn_session_choose_allowed(rn_session* session, const uint8_t* allowed, rn_choice* out);
/* The stream the session's work runs on (hipStream_t as void*). */
int rn_session_stream(const rn_session* session, void** stream);

/* Per-kernel timing of greedy decode steps (no reference counterpart: the
 * reference has no tracing; it is this library's tracing hook). Runs `steps`
 * greedy steps like rn_session_decode_greedy, launching the step's kernels
 * directly with a HIP event after each, and returns for every kernel kind the
 * average microseconds per launch (kind_us) and launches per step (kind_count),
 * both arrays of RN_PROFILE_KINDS entries in this order: */
enum {
    RN_PROFILE_QKV_ATTENTION = 0, /* norm + each head's q/k/v rows + rotary + fp16 append + attention
                                     (layer 0: + the previous step's argmax and the embedding), one
                                     block per head */
    RN_PROFILE_OUT = 1,           /* quantise + out product + residual */
    RN_PROFILE_GATE_UP = 2,       /* norm + gate/up product + silu(gate)*up */
    RN_PROFILE_DOWN = 3,          /* quantise + down product + residual */
    RN_PROFILE_LOGITS = 4,        /* final norm + tied logits product + per-block argmax keys + position
                                     advance (the next step's first kernel reduces the keys) */
    RN_PROFILE_FINAL = 5,         /* a separate argmax reduction (0 launches a step in this build) */
    RN_PROFILE_KINDS = 6
};
int rn_session_profile_step(rn_session* session, uint32_t first, int steps, float* kind_us, int* kind_count);

/* ---- batched decode: `count` independent sequences advanced together --------- */
/* Like `count` Sessions, but each step runs the products as M=count i8-MFMA
 * GEMMs and the attention over `count` ragged caches in one launch. */
int rn_batch_create(const rn_model* model, int count, int capacity, rn_batch** out);
int rn_batch_free(rn_batch* batch);
int rn_batch_set_cache(rn_batch* batch, int sequence, int length, const uint16_t* keys,
                       const uint16_t* values);
/* ids [count][steps] (host out). */
int rn_batch_decode_greedy(rn_batch* batch, const uint32_t* first, int steps, uint32_t* ids);
/* Per-sequence rn_session_truncate: lengths [count], each <= its current length. */
int rn_batch_truncate(rn_batch* batch, const int32_t* lengths);
/* Session::logits (session.rs:166-177) of every sequence after the last
 * decoded step: out [count][vocab] (host). RN_ERR_STATE before any step. */
int rn_batch_logits(const rn_batch* batch, float* out);
/* rn_session_get_cache for one sequence: the first `length` (<= its length)
 * cached positions, [layers][heads][length][head_dim] fp16 bits (host out). */
int rn_batch_get_cache(const rn_batch* batch, int sequence, int length, uint16_t* keys, uint16_t* values);
int rn_batch_stream(const rn_batch* batch, void** stream);

/* ---- Whistle-style speech path (crates/whistle) -------------------------------- */
/* The configuration: a stem of two conv1d layers (stem.rs:39-115 in one
 * dimension of time: an fp32 conv mels -> d, kernel 3 stride 1 + silu, then a
 * conv d -> d, kernel 3 stride 2, as an int8 product over im2col rows of three
 * frames + silu) to (frames - 1) / 2 + 1 encoder frames; encoder layers
 * of int8 self-attention (encoder.rs:217-297) and a gated FFN; a decoder of
 * the Session kind with cross-attention after each self-attention
 * (session.rs:126-128, cross.rs:126-182); tied int8 logits. d_model 384 or
 * 512 with heads of 64, ffn in {512, 1024, 1536, 2048}, mels <= 128, at most
 * 3072 mel frames (1536 encoder frames). */
typedef struct {
    int mels, frames, d_model, heads, head_dim, enc_layers, dec_layers, ffn, vocab, max_positions, group;
    float rope_theta, norm_eps;
} rn_whistle_config;
typedef struct rn_whistle rn_whistle;

/* The front end (crates/whistle/src/frontend.rs): Frontend::new (frontend.rs:31-40)
 * with the archive's mel filterbank [fft_size/2 + 1][mels] (host floats); the
 * Hann window and FFT twiddles are built on the host in float from cosf/sinf.
 * fft_size a power of two <= 4096, mels <= 256. */
typedef struct rn_frontend rn_frontend;
int rn_frontend_create(int mels, int fft_size, int window, int hop, const float* mel_weights, rn_frontend** out);
int rn_frontend_free(rn_frontend* frontend);
/* Frontend::log_mel (frontend.rs:72-102) on the device: samples (host, n) ->
 * features (host, [n/hop + 1][mels]) normalised per mel over the valid
 * frames (frames past them 0), *frames = n/hop + 1, *valid = n/hop, *spread
 * (Frontend::spread of the un-normalised log-mel, frontend.rs:104-116). The FFT,
 * power spectrum, mel sums and normalisation follow the reference's float
 * order; ln is the device logf where the reference calls the host libm's, so
 * features agree with it within 5e-5 (1 + |x|), not bit for bit. */
int rn_frontend_log_mel(rn_frontend* frontend, const float* samples, int n, float* features, int* frames,
                        int* valid, float* spread);

/* Host weights of the speech model (int8 codes with fp32 per-32 scales, fp32
 * gains; every pointer host memory, copied at creation). */
typedef struct {
    rn_qmat_host qkv;                  /* [3 d][d]: q rows, k rows, v rows */
    rn_qmat_host out;                  /* [d][d] */
    rn_qmat_host gate_up;              /* [2 ffn][d] */
    rn_qmat_host down;                 /* [d][ffn] */
    const float *norm_attn, *norm_ffn; /* [d] */
    const float *q_norm, *k_norm;      /* [64] per-head gains (encoder.rs:226-244) */
} rn_whistle_enc_host;
typedef struct {
    rn_qmat_host qkv, out;             /* self-attention, as the encoder's */
    rn_qmat_host cross_q;              /* [d][d] */
    rn_qmat_host cross_kv;             /* [2 d][d]: key rows, then value rows of the memory */
    rn_qmat_host cross_out;            /* [d][d] */
    rn_qmat_host gate_up, down;
    const float *norm_attn, *norm_cross, *post_norm, *norm_ffn; /* [d] */
    const float *q_norm, *k_norm;      /* [64] cross-attention head gains */
    float gate;                        /* the layer gate; the residual gain is sigmoid(gate) (cross.rs:178) */
} rn_whistle_dec_host;
typedef struct {
    const float* conv1;                /* [d][3][mels] fp32 */
    rn_qmat_host conv2;                /* [d][3 d]: column k d + i is tap k of input channel i */
    const rn_whistle_enc_host* enc;    /* [enc_layers] */
    const float* enc_norm;             /* [d] */
    float position_gate;               /* the cross position term's gain is sigmoid(position_gate) (cross.rs:61-72) */
    rn_qmat_host embedding;            /* [vocab][d], tied with the logits */
    const rn_whistle_dec_host* dec;    /* [dec_layers] */
    const float* dec_norm;             /* [d] */
} rn_whistle_weights_host;

/* Whistle::open (lib.rs:101-140) over host weights: the model, its work
 * buffers and one decoder session of max_positions positions, on their own
 * stream. */
int rn_whistle_create(const rn_whistle_config* config, const rn_whistle_weights_host* weights, rn_whistle** out);
/* The same with seeded synthetic weights drawn by name (the same draws as
 * rn_synth_*). */
int rn_whistle_create_synthetic(const rn_whistle_config* config, uint64_t seed, rn_whistle** out);
int rn_whistle_free(rn_whistle* whistle);
/* Encoder frames (frames - 1) / 2 + 1 (stem.rs:23-25). */
int rn_whistle_frames(const rn_whistle* whistle, int* frames);
/* The host-computed tables: the cross position term [frames][d_model]
 * (cross.rs:61-72) and the per-decoder-layer cross gains sigmoid(gate)
 * (cross.rs:178); both nullable. */
int rn_whistle_tables(const rn_whistle* whistle, float* position, float* cross_gains);
/* Stem::forward (stem.rs:39-115) alone: mel [frames][mels] -> out [T][d]. */
int rn_whistle_stem(rn_whistle* whistle, const float* mel, float* out);
/* Whistle::encode (lib.rs:155-161) then CrossWeights::memory (cross.rs:58-99):
 * the encoded frames and every decoder layer's int8 key/value memory stay on
 * the device; `encoded` (nullable) receives [T][d]. Resets the decoder. */
int rn_whistle_encode(rn_whistle* whistle, const float* mel, float* encoded);
/* Whistle::encode from samples (lib.rs:155-161): Frontend::log_mel
 * (frontend.rs:72-103) runs on the device and the stem reads its features in
 * place, with no round trip through the host; then as rn_whistle_encode.
 * samples: n host floats with n / hop == the model's frames; the front end's
 * mels must be the model's. spread (nullable) receives Features::spread. */
int rn_whistle_encode_samples(rn_whistle* whistle, const rn_frontend* frontend, const float* samples, int n,
                              float* encoded, float* spread);
/* The cross memory of the last encode: keys/values [dec_layers][T][heads][64]
 * int8, scales [dec_layers][T][heads]. */
int rn_whistle_memory(const rn_whistle* whistle, int8_t* keys, float* key_scales, int8_t* values,
                      float* value_scales);
/* Session::new for the decoder (an empty self-attention cache). */
int rn_whistle_reset(rn_whistle* whistle);
/* Session::push_with(token, Some(cross)) (session.rs:76-148). */
int rn_whistle_push(rn_whistle* whistle, uint32_t token);
/* Session::logits (session.rs:166-177) after the last push (host out, vocab). */
int rn_whistle_logits(rn_whistle* whistle, float* out);
/* The decode loop of Whistle::decode (lib.rs:240-295) without language,
 * keywords or timestamps: token = first; `steps` times { push; token =
 * argmax(logits); ids[i] = token }, the argmax on the device. */
int rn_whistle_decode_greedy(rn_whistle* whistle, uint32_t first, int steps, uint32_t* ids);
int rn_whistle_stream(const rn_whistle* whistle, void** stream);

/* ---- seeded synthetic inputs (host memory; no reference counterpart) ---------- */
/* SplitMix64 stream per tensor: state0 = seed ^ FNV-1a-64(name). */
int rn_synth_codes(uint64_t seed, const char* name, int8_t* out, size_t n);  /* U{-127..127} */
int rn_synth_uniform(uint64_t seed, const char* name, float lo, float hi, float* out, size_t n);
int rn_synth_normal(uint64_t seed, const char* name, float sigma, float* out, size_t n);
int rn_synth_normal_f16(uint64_t seed, const char* name, uint16_t* out, size_t n);
int rn_synth_tokens(uint64_t seed, const char* name, uint32_t vocab, uint32_t* out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
