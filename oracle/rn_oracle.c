/*
 * rn_oracle.c — CPU oracle for the Needle token loop (test infrastructure only;
 * see rn_oracle.h for the canonical reduction trees and who may use this file).
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off -fopenmp). No fast-math:
 * every division and square root is IEEE correctly rounded.
 */
#include "rn_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void ro_set_threads(int threads) { g_threads = threads < 1 ? 1 : threads; }
int ro_get_threads(void) { return g_threads; }

/* ---- scalar primitives ----------------------------------------------------- */

/* ops.rs:82-90: clamp to [-87, 87], scale by log2(e), round half away from zero,
 * degree-5 Horner polynomial in the fraction, times 2^whole built from bits. */
float ro_fast_exp(float value) {
    const float log2e = 1.44269504088896340736f;
    const float ln2 = 0.693147180559945309417f;
    float clamped = value < -87.0f ? -87.0f : (value > 87.0f ? 87.0f : value);
    float scaled = clamped * log2e;
    float whole = roundf(scaled);
    float f = scaled - whole;
    float p = 1.0f + f * (ln2 + f * (0.2402265f + f * (0.05550411f + f * (0.009618129f + f * 0.0013333558f))));
    int exponent = (int)whole + 127;
    uint32_t bits = (uint32_t)exponent << 23;
    float scale;
    memcpy(&scale, &bits, sizeof scale);
    return p * scale;
}

/* ops.rs:73-76 */
float ro_silu(float value) { return value / (1.0f + ro_fast_exp(-value)); }

/* f32::exp and ops::sigmoid (ops.rs:68-71) over arrays: the C library's expf,
 * which the reference's f32::exp calls. */
void ro_libm_exp_array(const float* x, float* y, size_t n, int sigmoid) {
#pragma omp parallel for schedule(static) num_threads(ro_get_threads())
    for (size_t i = 0; i < n; ++i) y[i] = sigmoid ? 1.0f / (1.0f + expf(-x[i])) : expf(x[i]);
}

/* f32::ln over an array: the C library's logf, which the reference's f32::ln
 * calls (frontend.rs:96-99). */
void ro_libm_log_array(const float* x, float* y, size_t n) {
#pragma omp parallel for schedule(static) num_threads(ro_get_threads())
    for (size_t i = 0; i < n; ++i) y[i] = logf(x[i]);
}

/* ops.rs:32-42 — max is order-free (NaN operands are ignored like f32::max). */
float ro_peak_magnitude(const float* x, int n) {
    float peak = 0.0f;
    for (int i = 0; i < n; ++i) peak = fmaxf(peak, fabsf(x[i]));
    return peak;
}

/* ops.rs:103-110 */
float ro_int8_scale(const float* x, int n) {
    float peak = ro_peak_magnitude(x, n);
    return peak > 0.0f ? peak / 127.0f : 1.0f;
}

/* round-half-even, clamp to [-128, 127], NaN -> 0 (Rust `as i8` saturates NaN to 0) */
static inline int8_t quantise_one(float value, float scale) {
    float q = rintf(value / scale);
    q = q < -128.0f ? -128.0f : (q > 127.0f ? 127.0f : q);
    if (q != q) return 0;
    return (int8_t)q;
}

/* ops.rs:112-118 */
float ro_quantise_int8(const float* x, int n, int8_t* codes) {
    float scale = ro_int8_scale(x, n);
    for (int i = 0; i < n; ++i) codes[i] = quantise_one(x[i], scale);
    return scale;
}

/* ops.rs:120-125 */
void ro_fake_quantise_int8(float* x, int n) {
    float scale = ro_int8_scale(x, n);
    for (int i = 0; i < n; ++i) {
        float q = rintf(x[i] / scale);
        q = q < -128.0f ? -128.0f : (q > 127.0f ? 127.0f : q);
        x[i] = q * scale;
    }
}

/* ops.rs:7-17 (tree T1): eight strided lanes, lanes summed in order, then the tail. */
float ro_sum_of_squares(const float* x, int n) {
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int chunks = n / 8;
    for (int c = 0; c < chunks; ++c)
        for (int j = 0; j < 8; ++j) {
            float v = x[8 * c + j];
            lanes[j] = lanes[j] + v * v;
        }
    float tail = 0.0f;
    for (int i = chunks * 8; i < n; ++i) tail = tail + x[i] * x[i];
    float total = 0.0f;
    for (int j = 0; j < 8; ++j) total = total + lanes[j];
    return total + tail;
}

/* ops.rs:44-50; eps 1e-6 as NORM_EPSILON at ops.rs:1 */
void ro_zero_centred_norm(const float* x, const float* gain, int n, float* out) {
    float mean_square = ro_sum_of_squares(x, n) / (float)n;
    float inverse = 1.0f / sqrtf(mean_square + 1e-6f);
    for (int i = 0; i < n; ++i) out[i] = ((1.0f + gain[i]) * x[i]) * inverse;
}

/* ops.rs:92-101 */
void ro_softmax_in_place(float* v, int n) {
    float peak = -INFINITY;
    for (int i = 0; i < n; ++i) peak = fmaxf(peak, v[i]);
    float total = 0.0f;
    for (int i = 0; i < n; ++i) {
        v[i] = ro_fast_exp(v[i] - peak);
        total = total + v[i];
    }
    float inverse = 1.0f / total;
    for (int i = 0; i < n; ++i) v[i] = v[i] * inverse;
}

/* ops.rs:127-129: 1 / theta^(2i/hd), all in f32 */
void ro_rotary_frequencies(int head_dim, float theta, float* freqs) {
    for (int i = 0; i < head_dim / 2; ++i)
        freqs[i] = 1.0f / powf(theta, (2.0f * (float)i) / (float)head_dim);
}

/* The angle of ops.rs:135 (position as f32 times the frequency) and its sin/cos,
 * tabulated once so that every consumer reads identical values. */
void ro_rotary_table(int head_dim, float theta, int positions, float* cos_tab, float* sin_tab) {
    int half = head_dim / 2;
    float* freqs = (float*)malloc(sizeof(float) * (size_t)half);
    ro_rotary_frequencies(head_dim, theta, freqs);
    for (int p = 0; p < positions; ++p)
        for (int i = 0; i < half; ++i) {
            float angle = (float)p * freqs[i];
            cos_tab[(size_t)p * half + i] = cosf(angle);
            sin_tab[(size_t)p * half + i] = sinf(angle);
        }
    free(freqs);
}

/* ops.rs:131-141: rotate-half pairs (i, i + hd/2). */
void ro_apply_rotary(float* head, int head_dim, const float* cos_row, const float* sin_row) {
    int half = head_dim / 2;
    for (int i = 0; i < half; ++i) {
        float a = head[i], b = head[i + half];
        float c = cos_row[i], s = sin_row[i];
        head[i] = a * c - b * s;
        head[i + half] = b * c + a * s;
    }
}

/* IEEE binary16 conversion, round to nearest even (subnormals and overflow handled). */
uint16_t ro_f32_to_f16(float value) {
    uint32_t x;
    memcpy(&x, &value, sizeof x);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7fffffffu;
    if (absx > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((absx >> 13) & 0x3ffu)); /* NaN */
    if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520: inf */
    if (absx < 0x38800000u) { /* below the smallest normal half: subnormal or zero */
        if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 (ties-even at 2^-25) */
        uint32_t mant = (absx & 0x7fffffu) | 0x800000u;
        int e = (int)(absx >> 23); /* 102..112 */
        int shift = 126 - e;       /* value = mant * 2^(e-150); half ulp units 2^-24 */
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1u))) q += 1;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (absx >> 23) - 112u; /* rebias 127 -> 15 */
    uint32_t mant = absx & 0x7fffffu;
    uint32_t q = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1; /* carries into exponent correctly */
    return (uint16_t)(sign | q);
}

/* binary16 -> binary32 is exact; F16C (x86-64-v3) does it in one instruction. */
static inline float half_to_float(uint16_t h) { return _cvtsh_ss(h); }

float ro_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t mant = (uint32_t)h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (mant == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int shift = 0;
            while ((mant & 0x400u) == 0) { mant <<= 1; ++shift; }
            mant &= 0x3ffu;
            bits = sign | ((uint32_t)(113 - shift) << 23) | (mant << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (mant << 13);
    }
    float out;
    memcpy(&out, &bits, sizeof out);
    return out;
}

/* generator.rs:257-265: first index of the strict maximum; a NaN never wins, and
 * a NaN at index 0 is never displaced (every comparison against it is false). */
uint32_t ro_argmax(const float* values, int n) {
    int best = 0;
    for (int i = 0; i < n; ++i)
        if (values[i] > values[best]) best = i;
    return (uint32_t)best;
}

/* ---- quantised products (tree T4) -------------------------------------------- */

/* One 32-code group: a constant trip count lets the compiler keep it in vector registers. */
static inline int32_t dot32(const int8_t* a, const int8_t* b) {
    int32_t s = 0;
    for (int k = 0; k < 32; ++k) s += (int32_t)a[k] * (int32_t)b[k];
    return s;
}

static void product_rows(int form, const int8_t* W, const float* sW, int cols, int group,
                         const int8_t* xq, const float* sx, int count, int rows, int n0, int n1,
                         float* y, int32_t* acc) {
    int groups = cols / group;
    for (int n = n0; n < n1; ++n) {
        const int8_t* wrow = W + (size_t)n * cols;
        const float* srow = sW + (size_t)n * groups;
        for (int t = 0; t < count; ++t) {
            const int8_t* xrow = xq + (size_t)t * cols;
            float total = 0.0f;
            for (int g = 0; g < groups; ++g) {
                int32_t a = 0;
                const int8_t* wg = wrow + g * group;
                const int8_t* xg = xrow + g * group;
                if (group == 32)
                    a = dot32(wg, xg);
                else
                    for (int k = 0; k < group; ++k) a += (int32_t)wg[k] * (int32_t)xg[k];
                if (acc) acc[((size_t)t * rows + n) * groups + g] = a;
                if (form == RO_FORM_PANEL) {
                    total = fmaf((float)a, srow[g] * sx[t], total);  /* panel.rs:184-188 */
                } else {
                    total = total + ((float)a * srow[g]) * sx[t];     /* neon.rs:180 */
                }
            }
            y[(size_t)t * rows + n] = total;
        }
    }
}

/* Rows fan out over threads in tasks of 64 rows once there are at least 512 row
 * products, following matrix.rs:9-10 and 155-165. Results do not depend on it. */
void ro_product(int form, const int8_t* W, const float* sW, int rows, int cols, int group,
                const int8_t* xq, const float* sx, int count, float* y, int32_t* acc) {
    const int task = 64;
    int tasks = (rows + task - 1) / task;
    if (g_threads > 1 && (long)rows * count >= 512) {
#pragma omp parallel for schedule(dynamic, 1) num_threads(g_threads)
        for (int i = 0; i < tasks; ++i) {
            int n0 = i * task, n1 = n0 + task < rows ? n0 + task : rows;
            product_rows(form, W, sW, cols, group, xq, sx, count, rows, n0, n1, y, acc);
        }
    } else {
        product_rows(form, W, sW, cols, group, xq, sx, count, rows, 0, rows, y, acc);
    }
}

void ro_multiply(int form, const int8_t* W, const float* sW, int rows, int cols, int group,
                 const float* x, int count, float* y, int32_t* acc, int8_t* codes, float* scales) {
    int8_t* xq = codes ? codes : (int8_t*)malloc((size_t)count * cols);
    float* sx = scales ? scales : (float*)malloc(sizeof(float) * (size_t)count);
    for (int t = 0; t < count; ++t) sx[t] = ro_quantise_int8(x + (size_t)t * cols, cols, xq + (size_t)t * cols);
    ro_product(form, W, sW, rows, cols, group, xq, sx, count, y, acc);
    if (!codes) free(xq);
    if (!scales) free(sx);
}

/* ---- attention (trees T2 and T3) --------------------------------------------- */

#define RO_SCORE_PARTS 16  /* T2: sub-sums of head_dim/16 consecutive dims */
#define RO_CLASSES 32      /* T3: interleaved position classes p mod 32 */

static float score_tree(const float* q, const uint16_t* k, int head_dim) {
    int per = head_dim / RO_SCORE_PARTS;
    float part[RO_SCORE_PARTS];
    for (int j = 0; j < RO_SCORE_PARTS; ++j) {
        float s = 0.0f;
        for (int i = 0; i < per; ++i) s = s + q[j * per + i] * half_to_float(k[j * per + i]);
        part[j] = s;
    }
    for (int width = 1; width < RO_SCORE_PARTS; width *= 2)
        for (int j = 0; j < RO_SCORE_PARTS; j += 2 * width) part[j] = part[j] + part[j + width];
    return part[0];
}

/* kernels/src/attention.rs:251-280 with float scores over an fp16 cache:
 * coefficient = score / sqrt(head_dim) (attention.rs:193,198), peak-subtracted
 * fast_exp weights, weighted values, then one multiply by 1/total. */
void ro_attend_head(const float* q, const uint16_t* K, const uint16_t* V, int head_dim, int length,
                    float* out) {
    float* c = (float*)malloc(sizeof(float) * (size_t)(length > 0 ? length : 1));
    float inverse_root = 1.0f / sqrtf((float)head_dim);
    float peak = -INFINITY;
    for (int p = 0; p < length; ++p) {
        c[p] = score_tree(q, K + (size_t)p * head_dim, head_dim) * inverse_root;
        peak = fmaxf(peak, c[p]);
    }
    for (int p = 0; p < length; ++p) c[p] = ro_fast_exp(c[p] - peak);
    float totals[RO_CLASSES];
    for (int j = 0; j < RO_CLASSES; ++j) {
        float t = 0.0f;
        for (int p = j; p < length; p += RO_CLASSES) t = t + c[p];
        totals[j] = t;
    }
    float total = 0.0f;
    for (int j = 0; j < RO_CLASSES; ++j) total = total + totals[j];
    float inverse = 1.0f / total;
    /* part[j][d] accumulates positions p = j, j+32, ... in increasing p. */
    float* part = (float*)calloc((size_t)RO_CLASSES * head_dim, sizeof(float));
    for (int p = 0; p < length; ++p) {
        float* acc = part + (size_t)(p % RO_CLASSES) * head_dim;
        const uint16_t* v = V + (size_t)p * head_dim;
        for (int d = 0; d < head_dim; ++d) acc[d] = acc[d] + c[p] * half_to_float(v[d]);
    }
    for (int d = 0; d < head_dim; ++d) {
        float o = 0.0f;
        for (int j = 0; j < RO_CLASSES; ++j) o = o + part[(size_t)j * head_dim + d];
        out[d] = o * inverse;
    }
    free(part);
    free(c);
}

/* ---- decoder ------------------------------------------------------------------- */

static size_t cache_offset(const ro_config* c, const ro_session* s, int layer, int head, int pos) {
    return (((size_t)layer * c->heads + head) * (size_t)s->capacity + (size_t)pos) * (size_t)c->head_dim;
}

/* Embedding row dequantised (matrix.rs:140-153 for int8 codes) times sqrt(d)
 * (session.rs:85-90). */
void ro_embed(const ro_config* c, const ro_model* m, uint32_t token, float* x) {
    int d = c->d_model, groups = d / c->group;
    const int8_t* row = m->embedding.codes + (size_t)token * d;
    const float* srow = m->embedding.scales + (size_t)token * groups;
    float root = sqrtf((float)d);
    for (int k = 0; k < d; ++k) x[k] = ((float)row[k] * srow[k / c->group]) * root;
}

/* Attention for `count` tokens at positions first..first+count-1 of one layer:
 * qkv rows are [count][3d] (already produced by the fused product); rotary,
 * fp16 append and attention per (token, head). Writes attended [count][d]. */
static void attention_layer(const ro_config* c, const ro_model* m, ro_session* s, int layer,
                            int first, int count, float* qkv, float* attended) {
    int d = c->d_model, hd = c->head_dim, half = hd / 2;
    for (int t = 0; t < count; ++t) {
        int pos = first + t;
        const float* cs = m->rope_cos + (size_t)pos * half;
        const float* sn = m->rope_sin + (size_t)pos * half;
        float* row = qkv + (size_t)t * 3 * d;
        for (int h = 0; h < c->heads; ++h) {
            ro_apply_rotary(row + h * hd, hd, cs, sn);
            ro_apply_rotary(row + d + h * hd, hd, cs, sn);
            size_t off = cache_offset(c, s, layer, h, pos);
            for (int i = 0; i < hd; ++i) {
                s->keys[off + i] = ro_f32_to_f16(row[d + h * hd + i]);
                s->values[off + i] = ro_f32_to_f16(row[2 * d + h * hd + i]);
            }
        }
    }
    int items = count * c->heads;
    int parallel = g_threads > 1 && first + 1 >= 128;  /* attention.rs:9,162-166 */
#pragma omp parallel for schedule(dynamic, 1) num_threads(g_threads) if (parallel)
    for (int item = 0; item < items; ++item) {
        int t = item / c->heads, h = item % c->heads;
        int pos = first + t;
        ro_attend_head(qkv + (size_t)t * 3 * d + h * hd, s->keys + cache_offset(c, s, layer, h, 0),
                       s->values + cache_offset(c, s, layer, h, 0), hd, pos + 1,
                       attended + (size_t)t * d + h * hd);
    }
}

/* One layer for `count` tokens held in x [count][d] (session.rs:109-138 and
 * prefill.rs:47-87 restated for the config's block: norm, fused QKV product,
 * rotary, fp16 append, attention, out product + residual, norm, fused
 * gate/up product, silu(gate)*up, down product + residual). */
static void layer_forward(const ro_config* c, const ro_model* m, ro_session* s, int layer, int first,
                          int count, float* x) {
    const ro_layer* L = &m->layers[layer];
    int d = c->d_model, f = c->ffn, g = c->group;
    float* h = (float*)malloc(sizeof(float) * (size_t)count * (2 * f > 3 * d ? 2 * f : 3 * d));
    float* y = (float*)malloc(sizeof(float) * (size_t)count * (2 * f > 3 * d ? 2 * f : 3 * d));
    float* normed = (float*)malloc(sizeof(float) * (size_t)count * d);

    for (int t = 0; t < count; ++t) ro_zero_centred_norm(x + (size_t)t * d, L->norm_attn, d, normed + (size_t)t * d);
    ro_multiply(RO_FORM_PANEL, L->qkv.codes, L->qkv.scales, 3 * d, d, g, normed, count, y, NULL, NULL, NULL);
    attention_layer(c, m, s, layer, first, count, y, h);
    ro_multiply(RO_FORM_PANEL, L->out.codes, L->out.scales, d, d, g, h, count, y, NULL, NULL, NULL);
    for (size_t i = 0; i < (size_t)count * d; ++i) x[i] = x[i] + y[i];

    for (int t = 0; t < count; ++t) ro_zero_centred_norm(x + (size_t)t * d, L->norm_ffn, d, normed + (size_t)t * d);
    ro_multiply(RO_FORM_PANEL, L->gate_up.codes, L->gate_up.scales, 2 * f, d, g, normed, count, y, NULL, NULL, NULL);
    for (int t = 0; t < count; ++t)
        for (int i = 0; i < f; ++i)
            h[(size_t)t * f + i] = ro_silu(y[(size_t)t * 2 * f + i]) * y[(size_t)t * 2 * f + f + i];
    ro_multiply(RO_FORM_PANEL, L->down.codes, L->down.scales, d, f, g, h, count, y, NULL, NULL, NULL);
    for (size_t i = 0; i < (size_t)count * d; ++i) x[i] = x[i] + y[i];

    free(h);
    free(y);
    free(normed);
}

static void run_tokens(const ro_config* c, const ro_model* m, ro_session* s, const uint32_t* tokens,
                       int count) {
    int d = c->d_model;
    float* x = (float*)malloc(sizeof(float) * (size_t)count * d);
    for (int t = 0; t < count; ++t) ro_embed(c, m, tokens[t], x + (size_t)t * d);
    int first = s->length;
    for (int l = 0; l < c->layers; ++l) layer_forward(c, m, s, l, first, count, x);
    s->length = first + count;
    ro_zero_centred_norm(x + (size_t)(count - 1) * d, m->norm_final, d, s->hidden);
    free(x);
}

void ro_session_push(const ro_config* c, const ro_model* m, ro_session* s, uint32_t token) {
    run_tokens(c, m, s, &token, 1);
}

void ro_session_prefill(const ro_config* c, const ro_model* m, ro_session* s, const uint32_t* tokens,
                        int count) {
    if (count > 0) run_tokens(c, m, s, tokens, count);
}

/* session.rs:166-177 for int8 codes: per-row quantisation of the final hidden
 * state, then the plane-form product with the tied embedding. */
void ro_session_logits(const ro_config* c, const ro_model* m, const ro_session* s, float* logits) {
    ro_multiply(RO_FORM_PLANE, m->embedding.codes, m->embedding.scales, c->vocab, c->d_model, c->group,
                s->hidden, 1, logits, NULL, NULL, NULL);
}

void ro_greedy(const ro_config* c, const ro_model* m, ro_session* s, uint32_t first, int steps,
               uint32_t* ids) {
    float* logits = (float*)malloc(sizeof(float) * (size_t)c->vocab);
    uint32_t token = first;
    for (int step = 0; step < steps; ++step) {
        ro_session_push(c, m, s, token);
        ro_session_logits(c, m, s, logits);
        token = ro_argmax(logits, c->vocab);
        ids[step] = token;
    }
    free(logits);
}
