/*
 * rn_oracle.h — CPU oracle for the Needle token loop (test infrastructure).
 *
 * This is NOT part of the product. It is a plain-C restatement of the reference
 * numerics (rustyneedle, crates/kernels, crates/model, crates/generate) at the
 * synthetic int8 configuration: int8 weight codes with one fp32 scale per
 * 32-element group along K, per-row int8 activation quantisation, an fp16 KV
 * cache, a single residual stream and a gated FFN. Only tests/, the smoke check
 * in __graft_entry__.py and the cpu_baseline leg of bench.py may load it, and
 * only as the checker or as the timed CPU baseline — never as the product path.
 *
 * Every float operation is written out in the order the kernels use; the file
 * is compiled with -ffp-contract=off so that `a * b + c` is two roundings and
 * `fmaf` is the only fused operation. Reductions whose order the reference
 * leaves platform-dependent (its NEON and x86 paths sum in different orders)
 * are fixed here as the canonical trees below, and the HIP kernels implement
 * exactly the same trees:
 *
 *   T1 sum of squares (RMSNorm): eight strided lanes, each summed in index
 *      order, lanes then added 0..7, then the tail — ops.rs:7-17 verbatim.
 *   T2 attention score q.k over head_dim = 16*c dims: sixteen sub-sums of c
 *      consecutive dims (each 0 + q0k0 + q1k1 + ... in order), then a balanced
 *      pairwise tree over the sixteen sub-sums in index order.
 *   T3 softmax total and P.V over L positions: thirty-two interleaved partial
 *      sums (position p goes to partial p mod 32, added in increasing p,
 *      starting from 0), then the partials added 0..31 starting from 0.
 *   T4 product epilogue per (token, row): sequential over groups g = 0..G-1.
 *      Panel form (layer matrices, panel.rs:184-188):
 *          total = fmaf((float)acc_g, sW[g] * sx, total)
 *      Plane form (tied embedding / logits, neon.rs:180):
 *          total = total + ((float)acc_g * sW[g]) * sx
 *   Integer accumulators are exact and therefore order-free.
 *
 * Parity pins (tests/test_oracle_*.py): integer accumulators against an int64
 * brute force; fast_exp and softmax against the reference's own bounds
 * (crates/kernels/tests/softmax.rs); quantisation against tie/clamp/zero
 * known answers; RMSNorm, rotary, attention and the decoder step against
 * float64 restatements within stated tolerances; argmax against the tie and
 * NaN rules of generator.rs:257-265.
 */
#ifndef RN_ORACLE_H
#define RN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar and vector primitives: crates/kernels/src/ops.rs ---------------- */
float ro_fast_exp(float value);                                     /* ops.rs:82-90   */
void ro_libm_exp_array(const float* x, float* y, size_t n, int sigmoid); /* f32::exp, ops.rs:68-71 */
void ro_libm_log_array(const float* x, float* y, size_t n);              /* f32::ln, frontend.rs:96-99 */
float ro_silu(float value);                                         /* ops.rs:73-76   */
float ro_peak_magnitude(const float* x, int n);                     /* ops.rs:32-42   */
float ro_int8_scale(const float* x, int n);                         /* ops.rs:103-110 */
float ro_quantise_int8(const float* x, int n, int8_t* codes);       /* ops.rs:112-118 */
void ro_fake_quantise_int8(float* x, int n);                        /* ops.rs:120-125 */
float ro_sum_of_squares(const float* x, int n);                     /* ops.rs:7-17    */
void ro_zero_centred_norm(const float* x, const float* gain, int n, float* out); /* ops.rs:44-50 */
void ro_softmax_in_place(float* v, int n);                          /* ops.rs:92-101  */
void ro_rotary_frequencies(int head_dim, float theta, float* freqs); /* ops.rs:127-129 */
/* cos/sin of position * freq[i] for every position < positions: [positions][head_dim/2] */
void ro_rotary_table(int head_dim, float theta, int positions, float* cos_tab, float* sin_tab);
void ro_apply_rotary(float* head, int head_dim, const float* cos_row, const float* sin_row); /* ops.rs:131-141 */
uint16_t ro_f32_to_f16(float value);
float ro_f16_to_f32(uint16_t bits);
uint32_t ro_argmax(const float* values, int n);                     /* generator.rs:257-265 */

/* ---- quantised products ------------------------------------------------------ */
enum { RO_FORM_PANEL = 0, RO_FORM_PLANE = 1 };
/* y[t*rows + n] for t < count; acc (nullable) is [count][rows][cols/group] int32. */
void ro_product(int form, const int8_t* W, const float* sW, int rows, int cols, int group,
                const int8_t* xq, const float* sx, int count, float* y, int32_t* acc);
/* quantise_int8 each of `count` input rows of `cols` floats, then ro_product.
 * codes (nullable) receives [count][cols], scales (nullable) [count]. */
void ro_multiply(int form, const int8_t* W, const float* sW, int rows, int cols, int group,
                 const float* x, int count, float* y, int32_t* acc, int8_t* codes, float* scales);

/* ---- attention over an fp16 cache (kernels/src/attention.rs:251-280 restated) -- */
/* q: head_dim floats (already rotated); K, V: [length][head_dim] fp16 bits. */
void ro_attend_head(const float* q, const uint16_t* K, const uint16_t* V, int head_dim, int length,
                    float* out);

/* ---- decoder model and session (crates/model/src/session.rs, prefill.rs) ------ */
typedef struct {
    int layers, d_model, heads, head_dim, ffn, vocab, group, max_positions;
    float rope_theta, norm_eps;
} ro_config;

typedef struct { const int8_t* codes; const float* scales; } ro_qmat;

typedef struct {
    ro_qmat qkv;      /* [3*d][d]  rows: q (heads*head_dim), k, v            */
    ro_qmat out;      /* [d][d]                                              */
    ro_qmat gate_up;  /* [2*ffn][d] rows: gate 0..ffn-1, up ffn..2*ffn-1      */
    ro_qmat down;     /* [d][ffn]                                            */
    const float* norm_attn;  /* [d] zero-centred gains */
    const float* norm_ffn;   /* [d] */
} ro_layer;

typedef struct {
    ro_qmat embedding;         /* [vocab][d], tied with the logits product */
    const float* norm_final;   /* [d] */
    const ro_layer* layers;    /* [layers] */
    const float* rope_cos;     /* [max_positions][head_dim/2] */
    const float* rope_sin;
} ro_model;

/* A session owns its caches: keys/values are [layers][heads][capacity][head_dim]
 * fp16 bits; hidden is [d_model]; length counts the cached positions. */
typedef struct {
    uint16_t* keys;
    uint16_t* values;
    float* hidden;
    int capacity;
    int length;
} ro_session;

void ro_embed(const ro_config* c, const ro_model* m, uint32_t token, float* x);
/* Session::push_with (session.rs:76-148) for the config's block. */
void ro_session_push(const ro_config* c, const ro_model* m, ro_session* s, uint32_t token);
/* Session::prefill (prefill.rs:10-99): the same per-token arithmetic, batched. */
void ro_session_prefill(const ro_config* c, const ro_model* m, ro_session* s,
                        const uint32_t* tokens, int count);
/* Session::logits (session.rs:166-177). */
void ro_session_logits(const ro_config* c, const ro_model* m, const ro_session* s, float* logits);
/* The greedy loop of generator.rs:199-230 without grammar: starting from
 * token = first, `steps` times { push(token); logits; token = argmax; record }.
 * The last recorded token is not pushed. */
void ro_greedy(const ro_config* c, const ro_model* m, ro_session* s, uint32_t first, int steps,
               uint32_t* ids);

/* Threads used by products and head-parallel attention (1 = scalar). */
void ro_set_threads(int threads);
int ro_get_threads(void);

/* ---- codebook weight format (rn_codebook.c) ----------------------------------
 * Packed 2-bit / 4-bit / ternary indices with fp16 group norms, rotated input
 * (walsh.rs, matrix.rs, neon.rs, panel.rs); bits 5 marks ternary crumbs. */
void ro_walsh_transform(float* v, int n);                                        /* walsh.rs:41-76 */
void ro_codebook_prepare(const float* x, int columns, int padded, int group, float* rotated); /* matrix.rs:123-138 */
int ro_codebook_levels(const float* codebook, int bits, int group, float levels[16]); /* matrix.rs:499-508 */
float ro_integer_levels(const float levels[16], int count, int8_t table[16]);    /* neon.rs:114-124 */
void ro_group_codes(const float* rotated, int n, int group, int8_t* codes, float* scales); /* panel.rs:52-66 */
void ro_codebook_product(const uint8_t* packed, const uint16_t* norms, int rows, int padded, int group,
                         int bits, const int8_t table[16], float lscale, const int8_t* xcodes,
                         const float* xscales, int count, float* y, int32_t* acc);
void ro_codebook_dequantise_row(const uint8_t* packed, const uint16_t* norms, int padded, int columns,
                                int group, int bits, const float levels[16], int row, float* out); /* matrix.rs:140-153 */
/* the float path: fill_rows_float (matrix.rs:427-440) and multiply_batch's
 * float tile (matrix.rs:356-378); any width 1-5, rotated [count][padded] in */
void ro_codebook_float_vector(const uint8_t* packed, const uint16_t* norms, int rows, int padded, int group, int bits,
                              const float levels[16], const float* rotated, int count, float* y);
void ro_codebook_float_batch(const uint8_t* packed, const uint16_t* norms, int rows, int padded, int group, int bits,
                             const float levels[16], const float* rotated, int count, float* y);

/* ---- speech front end (rn_frontend.c): crates/whistle/src/frontend.rs ---------- */
void ro_frontend_tables(int fft_size, int window, float* win, float* twiddle_cos, float* twiddle_sin); /* :32-39 */
void ro_power_spectrum(float* real, float* imaginary, int size, const float* twiddle_cos, const float* twiddle_sin,
                       float* power);                                                                  /* :42-70 */
int ro_log_mel_raw(const float* samples, int n, int mels, int fft_size, int window, int hop,
                   const float* mel_weights, float* data);
float ro_spread(const float* data, int valid, int mels);                                               /* :104-116 */
void ro_normalise(float* data, int frames, int valid, int mels);                                       /* :118-133 */
int ro_log_mel(const float* samples, int n, int mels, int fft_size, int window, int hop, const float* mel_weights,
               float* data, int* valid, float* spread);                                                /* :72-102 */

/* ---- Kronecker apply (rn_hadamard.c): ops.rs:220-297, 32 x 32 factors ---------- */
void ro_kronecker_apply_32(const float* input, const float* left, const float* right, float* output);

/* ---- lanes hyper-connection (rn_lanes.c): crates/model/src/lanes.rs ------------ */
void ro_unit_rms(const float* x, int n, float* out);                                   /* ops.rs:60-66 */
void ro_sinkhorn(float* m, int size, int iterations);                                   /* ops.rs:198-217 */
void ro_lanes_route_tail(int lanes, int width, int layer, int slot, const float* a_pre, const float* a_post,
                         const float* a_res, const float* b_pre, const float* b_post, const float* b_res,
                         const float* stream, const float* pre, float* post, float* residual, float* input);
void ro_lanes_combine(int lanes, int width, const float* post, const float* residual, const float* stream,
                      const float* delta, float* next);                                 /* lanes.rs:86-98 */

/* ---- grammar-constrained choice (rn_generate.c) ------------------------------ */
int32_t ro_argmax_allowed(const float* values, const uint8_t* allowed, int n);   /* generator.rs:147-155 */
void ro_allowed_statistics(const float* logits, const uint8_t* allowed, int n, int token, float* probability,
                           float* mass);                                         /* generator.rs:182-194 */

/* ---- Whistle-style speech path (rn_whistle.c) ---------------------------------
 * crates/whistle: stem (stem.rs), encoder (encoder.rs), cross-attention
 * memory and apply (cross.rs), and the decoder step with the cross hook
 * (session.rs:76-148). The synthetic configuration keeps one residual stream
 * and a gated FFN, like the decoder above: stem = two conv1d layers, fp32
 * conv (mels -> d, k3, s1, pad 1) + silu, then conv (d -> d, k3, s2, pad 1)
 * as an int8 product over the im2col rows (three consecutive frames, each
 * row quantised per row) + silu; encoder layer = x += out(int8 attention over
 * all frames of norm(x)), x += down(silu(gate) * up) of norm(x); final norm. */
typedef struct {
    int mels, frames, d_model, heads, head_dim, enc_layers, dec_layers, ffn, vocab, max_positions, group;
    float rope_theta, norm_eps;
} ro_wconfig;

typedef struct {
    ro_qmat qkv, out, gate_up, down;
    const float *norm_attn, *norm_ffn;
    const float *q_norm, *k_norm; /* [head_dim] per-head gains */
} ro_wenc_layer;

typedef struct {
    ro_qmat qkv, out;           /* self-attention */
    ro_qmat cross_q;            /* [d][d] */
    ro_qmat cross_kv;           /* [2d][d]: key rows, then value rows, of the memory */
    ro_qmat cross_out;          /* [d][d] */
    ro_qmat gate_up, down;
    const float *norm_attn, *norm_cross, *post_norm, *norm_ffn;
    const float *q_norm, *k_norm; /* [head_dim] cross-attention head gains */
    float cross_gain;           /* sigmoid(layer gate), cross.rs:178 */
} ro_wdec_layer;

typedef struct {
    const float* conv1;          /* [d][3][mels] */
    ro_qmat conv2;               /* [d][3 d]: column k d + i is tap k of input channel i */
    const ro_wenc_layer* enc;
    const float* enc_norm;       /* [d] */
    const float* cross_position; /* [encoder frames][d]: sigmoid(gate) * sinusoid (cross.rs:61-72) */
    ro_qmat embedding;           /* [vocab][d], tied */
    const ro_wdec_layer* dec;
    const float* dec_norm;       /* [d] */
    const float* rope_cos;       /* [max(encoder frames, max_positions)][head_dim/2] */
    const float* rope_sin;
} ro_wmodel;

/* Cross memory [dec_layers][frames][heads][head_dim] int8 codes with
 * [dec_layers][frames][heads] scales; the self-attention cache as ro_session. */
typedef struct {
    uint16_t* keys;
    uint16_t* values;
    const int8_t* mem_k;
    const float* mem_ks;
    const int8_t* mem_v;
    const float* mem_vs;
    float* hidden;
    int capacity, length, frames;
} ro_wsession;

int ro_whistle_frames(const ro_wconfig* c); /* (frames - 1) / 2 + 1 (stem.rs:21-23) */
/* ops.rs:68-71 with the platform expf. */
float ro_sigmoid(float value);
/* cross.rs:61-72: gate * sin / cos of t * exp(rate * j) for frames 0..T-1, the
 * sines in columns 0..d/2-1 and the cosines in d/2..d-1, rate = -ln(10000)/(d/2 - 1). */
void ro_whistle_position_table(int T, int d, float gate, float* out);
/* Stem::forward for the synthetic stem: mel [frames][mels] -> out [T][d]. */
void ro_whistle_stem(const ro_wconfig* c, const ro_wmodel* m, const float* mel, float* out);
/* One encoder layer over x [T][d] in place. */
void ro_whistle_encoder_layer(const ro_wconfig* c, const ro_wmodel* m, int layer, float* x, int T);
/* Whistle::encode: stem, the encoder layers, the final norm -> out [T][d]. */
void ro_whistle_encode(const ro_wconfig* c, const ro_wmodel* m, const float* mel, float* out);
/* CrossWeights::memory (cross.rs:58-99): per decoder layer, keys and values of
 * the encoded frames (position added, quantised per row, key head norm) as int8
 * codes per (frame, head) with their scales. */
void ro_whistle_memory(const ro_wconfig* c, const ro_wmodel* m, const float* encoded, int T, int8_t* mem_k,
                       float* mem_ks, int8_t* mem_v, float* mem_vs);
/* One query head against `frames` int8 key/value rows (encoder.rs:266-285,
 * cross.rs:147-170): scores ((float)dot * key_scale) * query_scale, fast_exp
 * softmax with the totals in tree T3, weights times value scales, value codes
 * summed in tree T3. Row j of keys/values starts at j * row_stride, its scales
 * at j * scale_stride. */
void ro_int8_attend(const int8_t* qc, float query_scale, const int8_t* kc, const float* ks, const int8_t* vc,
                    const float* vs, int frames, int head_dim, int row_stride, int scale_stride, float* out);
/* Session::push_with with the cross hook (session.rs:76-148, cross.rs:126-182). */
void ro_whistle_push(const ro_wconfig* c, const ro_wmodel* m, ro_wsession* s, uint32_t token);
void ro_whistle_logits(const ro_wconfig* c, const ro_wmodel* m, const ro_wsession* s, float* logits);
void ro_whistle_greedy(const ro_wconfig* c, const ro_wmodel* m, ro_wsession* s, uint32_t first, int steps,
                       uint32_t* ids);

/* ---- Needle 3 (rn_needle3.c): crates/model/src, crates/cact/src --------------- */
/* A codebook matrix (QuantisedMatrix, matrix.rs:14-59) over the archive's blob. */
typedef struct {
    const uint8_t* packed;
    const uint16_t* norms;
    int rows, columns, padded, group, bits, groups;
    size_t row_bytes;
    float levels[16];
    int8_t table[16];
    float lscale;
    int integer; /* the integer path (2-, 4-bit, ternary) */
} ro_cbm;
void ro_cbm_init(ro_cbm* m, const uint8_t* blob, int rows, int columns, int group, int bits, const float* codebook);
void ro_cbm_prepare(const ro_cbm* m, const float* x, float* rotated);                    /* matrix.rs:123-128 */
void ro_cbm_rows(const ro_cbm* m, int first, int n, const float* rotated, float* y);    /* matrix.rs:402-421 */
void ro_cbm_dequantise_row(const ro_cbm* m, int row, float* out);                       /* matrix.rs:140-153 */

typedef struct { /* ModelConfig (config.rs:17-35) */
    int vocab, output_vocab, d_model, num_heads, num_kv_heads, num_layers, qk_head_dim, v_head_dim, max_seq_len;
    int lanes, sliding_window, conv_taps, hadamard_size;
    uint64_t global_layers;
    float rope_theta;
    int engram_slots, engram_sub_dim, engram_tables, engram_conv_taps, engram_dilation, engram_seed_heads;
    int engram_order_count, engram_orders[4], engram_heads_per_order, engram_site_count, engram_sites[16];
} ro_n3_config;
typedef struct { /* HadamardWeights (hadamard.rs:8-21) */
    int size, rank;
    float *d1, *d2, *b2, *d3, *d4, *cond_v, *cond_u;
    float* factors[6]; /* w1a w1b w2a w2b w3a w3b */
    int factor_sizes[6];
} ro_n3_hadamard;
typedef struct { /* LayerWeights + AttentionWeights (weights.rs:11-18, attention.rs:11-20) */
    float *norm_in, *q_norm, *k_norm, *post_norm, *pre_hadamard_norm;
    float attention_gate;
    float* taps[3];
    ro_cbm q, k, v, gate, out;
    ro_n3_hadamard hadamard;
} ro_n3_layer;
typedef struct { ro_cbm tables, key, value; float* taps; } ro_n3_engram; /* engram.rs:13-18 */
typedef struct { /* ProbeHead after with_rows (heads.rs:6-18) */
    int code, layers, probes_per_layer, queries, width;
    float *probes, *gain, *query, *row_bias, *bias;
    ro_cbm projection;
} ro_n3_head;
typedef struct {
    ro_n3_config config;
    float codebook[28];
    void* records;
    ro_cbm embedding;
    ro_n3_layer* layers;
    float *a_pre, *a_post, *a_res, *b_pre, *b_post, *b_res;
    ro_cbm phi_pre, phi_post, phi_res;
    int32_t* permutations[2];
    ro_n3_engram* engrams;
    float* final_norm;
    ro_n3_head* heads;
    int head_count;
    int* active;
    int active_count;
} ro_n3_model;
typedef struct { /* AttentionCache (attention.rs:36-44), dense: keys [cap][kv][qk], scales [kv][cap] */
    int8_t *keys, *values;
    float *key_scales, *value_scales;
    float* history; /* [conv_taps][q | k | v] newest first */
    int history_count, length;
} ro_n3_cache;
typedef struct {
    const ro_n3_model* m;
    int length, capacity;
    uint32_t* tokens;
    ro_n3_cache* caches;
    float** engram_history;
    int* engram_count;
    float *cos_tab, *sin_tab;
    float *hidden, *cells;
    float **peak, **total, **weighted;
} ro_n3_session;
/* Model::open over archive bytes (kept by the caller), then with_depth (depth
 * <= 0: every layer). 0, -1 malformed or unsupported, -2 depth outside the ladder. */
int ro_n3_open(const uint8_t* bytes, size_t size, int depth, ro_n3_model** out);
void ro_n3_close(ro_n3_model* m);
const ro_n3_config* ro_n3_config_of(const ro_n3_model* m);
int ro_n3_active(const ro_n3_model* m, int* layers);
int ro_n3_session_new(const ro_n3_model* m, int capacity, ro_n3_session** out);
void ro_n3_session_free(ro_n3_session* s);
int ro_n3_session_clone(const ro_n3_session* s, ro_n3_session** out);              /* session.rs:17 */
void ro_n3_push(ro_n3_session* s, uint32_t token);                                  /* session.rs:76-148 */
void ro_n3_feed(ro_n3_session* s, const uint32_t* tokens, int count);               /* session.rs:56-70 */
void ro_n3_logits(const ro_n3_session* s, float* logits);                           /* session.rs:151-165 */
int ro_n3_pooled_readout(const ro_n3_session* s, int code, float* pooled);          /* heads.rs:99-125 */
int ro_n3_head_output(const ro_n3_session* s, int code, float* out);                /* heads.rs:127-136 */
void ro_n3_table_indices(const ro_n3_config* c, const uint32_t* tokens, int position, int* indices); /* engram.rs:30-46 */
void ro_n3_hadamard_apply(const ro_n3_hadamard* h, const int32_t* first_perm, const int32_t* second_perm,
                          const float* input, int width, float* output);            /* hadamard.rs:55-107 */
void ro_n3_hadamard_arrays(int size, int rank, const float* d1, const float* d2, const float* b2, const float* d3,
                           const float* d4, const float* factors, const float* cond_v, const float* cond_u,
                           const int32_t* first_perm, const int32_t* second_perm, const float* input, int width,
                           float* output);
void ro_n3_attend_head(const int8_t* query, float query_scale, const int8_t* keys, const float* key_scales,
                       const int8_t* values, const float* value_scales, int count, int qk, int vd, int key_stride,
                       int value_stride, float* out);                                /* kernels/src/attention.rs:53-80 */

#ifdef __cplusplus
}
#endif
#endif
