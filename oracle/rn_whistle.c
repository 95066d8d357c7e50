/* rn_whistle.c — CPU restatement of the Whistle-style speech path: test
 * infrastructure, not the product (see rn_oracle.h for who may use it).
 *
 * Follows crates/whistle/src/stem.rs (stem stage), encoder.rs (attention with
 * int8 queries/keys/values), cross.rs (memory and apply) and the cross hook of
 * crates/model/src/session.rs:76-148, for the synthetic configuration declared
 * in rn_oracle.h. Float reductions use the fixed orders of rn_oracle.c: sums
 * of squares T1, the product epilogue T4, and T3 (32 interleaved position
 * classes) for every softmax total and weighted sum over frames. */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "rn_oracle.h"

#define RO_CLASSES 32

int ro_whistle_frames(const ro_wconfig* c) { return (c->frames > 1 ? c->frames - 1 : 0) / 2 + 1; }

static float* fbuf(size_t n) { return (float*)malloc(sizeof(float) * (n ? n : 1)); }

float ro_sigmoid(float value) { return 1.0f / (1.0f + expf(-value)); }

void ro_whistle_position_table(int T, int d, float gate, float* out) {
    const int half = d / 2;
    const float rate = -logf(10000.0f) / ((float)half - 1.0f);
    for (int t = 0; t < T; ++t)
        for (int j = 0; j < half; ++j) {
            float angle = (float)t * expf(rate * (float)j);
            out[(size_t)t * d + j] = gate * sinf(angle);
            out[(size_t)t * d + half + j] = gate * cosf(angle);
        }
}

/* The stem as two conv1d layers (stem.rs:39-115 keeps the reference's order of
 * operations: convolution, silu after each stage, an int8 product for the
 * learned projection). The first convolution adds taps (k, m) in that order
 * into a zero output, then silu. The second is the int8 product of conv2 with
 * the im2col rows: row t is frames 2t-1, 2t, 2t+1 of the first output (zero
 * outside the input), quantised per row like every product input; then silu. */
void ro_whistle_stem(const ro_wconfig* c, const ro_wmodel* m, const float* mel, float* out) {
    const int F = c->frames, M = c->mels, d = c->d_model, T = ro_whistle_frames(c);
    float* h1 = fbuf((size_t)F * d);
    int threads = ro_get_threads();
#pragma omp parallel for schedule(static) num_threads(threads) if (threads > 1)
    for (int t = 0; t < F; ++t) {
        for (int ch = 0; ch < d; ++ch) {
            float acc = 0.0f;
            for (int k = 0; k < 3; ++k) {
                int src = t + k - 1;
                if (src < 0 || src >= F) continue;
                const float* x = mel + (size_t)src * M;
                const float* w = m->conv1 + ((size_t)ch * 3 + k) * M;
                for (int i = 0; i < M; ++i) acc = acc + x[i] * w[i];
            }
            h1[(size_t)t * d + ch] = ro_silu(acc);
        }
    }
    float* cols = fbuf((size_t)T * 3 * d);
    for (int t = 0; t < T; ++t)
        for (int k = 0; k < 3; ++k) {
            const int src = 2 * t + k - 1;
            float* dst = cols + ((size_t)t * 3 + k) * d;
            if (src < 0 || src >= F)
                memset(dst, 0, sizeof(float) * (size_t)d);
            else
                memcpy(dst, h1 + (size_t)src * d, sizeof(float) * (size_t)d);
        }
    ro_multiply(RO_FORM_PANEL, m->conv2.codes, m->conv2.scales, d, 3 * d, c->group, cols, T, out, NULL, NULL, NULL);
    for (size_t i = 0; i < (size_t)T * d; ++i) out[i] = ro_silu(out[i]);
    free(cols);
    free(h1);
}

/* Per-head preparation (encoder.rs:226-263, cross.rs:86-97 and 149-156): the
 * zero-centred norm with the head gains (when given), the rotary at the
 * frame's position (when given), then quantise_int8. Returns the scale. */
static float head_codes(float* h, int hd, const float* gain, const float* cos_row, const float* sin_row,
                        int8_t* codes) {
    float tmp[256];
    if (gain) {
        ro_zero_centred_norm(h, gain, hd, tmp);
        memcpy(h, tmp, sizeof(float) * (size_t)hd);
    }
    if (cos_row) ro_apply_rotary(h, hd, cos_row, sin_row);
    return ro_quantise_int8(h, hd, codes);
}

void ro_int8_attend(const int8_t* qc, float query_scale, const int8_t* kc, const float* ks, const int8_t* vc,
                    const float* vs, int frames, int head_dim, int row_stride, int scale_stride, float* out) {
    float* e = fbuf((size_t)frames);
    float peak = -INFINITY;
    for (int j = 0; j < frames; ++j) {
        const int8_t* k = kc + (size_t)j * row_stride;
        int32_t dot = 0;
        for (int i = 0; i < head_dim; ++i) dot += (int32_t)qc[i] * (int32_t)k[i];
        e[j] = ((float)dot * ks[(size_t)j * scale_stride]) * query_scale;
        peak = fmaxf(peak, e[j]);
    }
    float part[RO_CLASSES];
    for (int j = 0; j < frames; ++j) e[j] = ro_fast_exp(e[j] - peak);
    for (int cl = 0; cl < RO_CLASSES; ++cl) {
        float t = 0.0f;
        for (int j = cl; j < frames; j += RO_CLASSES) t = t + e[j];
        part[cl] = t;
    }
    float total = 0.0f;
    for (int cl = 0; cl < RO_CLASSES; ++cl) total = total + part[cl];
    float inverse = 1.0f / total;
    /* ops.rs:99-100 weights, then encoder.rs:281 scale = value_scale * weight */
    for (int j = 0; j < frames; ++j) e[j] = vs[(size_t)j * scale_stride] * (e[j] * inverse);
    float* acc = (float*)calloc((size_t)RO_CLASSES * head_dim, sizeof(float));
    for (int j = 0; j < frames; ++j) {
        float* a = acc + (size_t)(j % RO_CLASSES) * head_dim;
        const int8_t* v = vc + (size_t)j * row_stride;
        for (int i = 0; i < head_dim; ++i) a[i] = a[i] + e[j] * (float)v[i];
    }
    for (int i = 0; i < head_dim; ++i) {
        float o = 0.0f;
        for (int cl = 0; cl < RO_CLASSES; ++cl) o = o + acc[(size_t)cl * head_dim + i];
        out[i] = o;
    }
    free(acc);
    free(e);
}

static void gated_ffn(const ro_wconfig* c, ro_qmat gate_up, ro_qmat down, const float* norm, float* x, int T) {
    const int d = c->d_model, f = c->ffn, g = c->group;
    float* normed = fbuf((size_t)T * d);
    float* y = fbuf((size_t)T * 2 * f);
    float* h = fbuf((size_t)T * f);
    for (int t = 0; t < T; ++t) ro_zero_centred_norm(x + (size_t)t * d, norm, d, normed + (size_t)t * d);
    ro_multiply(RO_FORM_PANEL, gate_up.codes, gate_up.scales, 2 * f, d, g, normed, T, y, NULL, NULL, NULL);
    for (int t = 0; t < T; ++t)
        for (int i = 0; i < f; ++i) h[(size_t)t * f + i] = ro_silu(y[(size_t)t * 2 * f + i]) * y[(size_t)t * 2 * f + f + i];
    ro_multiply(RO_FORM_PANEL, down.codes, down.scales, d, f, g, h, T, y, NULL, NULL, NULL);
    for (size_t i = 0; i < (size_t)T * d; ++i) x[i] = x[i] + y[i];
    free(h);
    free(y);
    free(normed);
}

/* encoder.rs:145-297 for the synthetic layer: norm, fused q/k/v product, per
 * head (q_norm | k_norm) + rotary at the frame position + int8 codes, values
 * quantised per head, attention of every frame over all frames, out product
 * + residual; then the gated FFN + residual. */
void ro_whistle_encoder_layer(const ro_wconfig* c, const ro_wmodel* m, int layer, float* x, int T) {
    const ro_wenc_layer* L = &m->enc[layer];
    const int d = c->d_model, H = c->heads, hd = c->head_dim, half = hd / 2, g = c->group;
    float* normed = fbuf((size_t)T * d);
    float* qkv = fbuf((size_t)T * 3 * d);
    for (int t = 0; t < T; ++t) ro_zero_centred_norm(x + (size_t)t * d, L->norm_attn, d, normed + (size_t)t * d);
    ro_multiply(RO_FORM_PANEL, L->qkv.codes, L->qkv.scales, 3 * d, d, g, normed, T, qkv, NULL, NULL, NULL);
    int8_t* qc = (int8_t*)malloc((size_t)T * d);
    int8_t* kc = (int8_t*)malloc((size_t)T * d);
    int8_t* vc = (int8_t*)malloc((size_t)T * d);
    float* qs = fbuf((size_t)T * H);
    float* ks = fbuf((size_t)T * H);
    float* vs = fbuf((size_t)T * H);
    const float inverse_root = 1.0f / sqrtf((float)hd);
    for (int t = 0; t < T; ++t) {
        const float* cs = m->rope_cos + (size_t)t * half;
        const float* sn = m->rope_sin + (size_t)t * half;
        float* row = qkv + (size_t)t * 3 * d;
        for (int h = 0; h < H; ++h) {
            size_t o = (size_t)t * d + (size_t)h * hd;
            qs[(size_t)t * H + h] = head_codes(row + h * hd, hd, L->q_norm, cs, sn, qc + o) * inverse_root;
            ks[(size_t)t * H + h] = head_codes(row + d + h * hd, hd, L->k_norm, cs, sn, kc + o);
            vs[(size_t)t * H + h] = head_codes(row + 2 * d + h * hd, hd, NULL, NULL, NULL, vc + o);
        }
    }
    float* context = fbuf((size_t)T * d);
    int threads = ro_get_threads();
#pragma omp parallel for schedule(dynamic, 4) num_threads(threads) if (threads > 1)
    for (int item = 0; item < T * H; ++item) {
        int t = item / H, h = item % H;
        ro_int8_attend(qc + (size_t)t * d + h * hd, qs[(size_t)t * H + h], kc + h * hd, ks + h, vc + h * hd, vs + h, T,
                       hd, d, H, context + (size_t)t * d + h * hd);
    }
    ro_multiply(RO_FORM_PANEL, L->out.codes, L->out.scales, d, d, g, context, T, qkv, NULL, NULL, NULL);
    for (size_t i = 0; i < (size_t)T * d; ++i) x[i] = x[i] + qkv[i];
    gated_ffn(c, L->gate_up, L->down, L->norm_ffn, x, T);
    free(context);
    free(vs);
    free(ks);
    free(qs);
    free(vc);
    free(kc);
    free(qc);
    free(qkv);
    free(normed);
}

void ro_whistle_encode(const ro_wconfig* c, const ro_wmodel* m, const float* mel, float* out) {
    const int d = c->d_model, T = ro_whistle_frames(c);
    float* x = fbuf((size_t)T * d);
    ro_whistle_stem(c, m, mel, x);
    for (int l = 0; l < c->enc_layers; ++l) ro_whistle_encoder_layer(c, m, l, x, T);
    for (int t = 0; t < T; ++t) ro_zero_centred_norm(x + (size_t)t * d, m->enc_norm, d, out + (size_t)t * d);
    free(x);
}

void ro_whistle_memory(const ro_wconfig* c, const ro_wmodel* m, const float* encoded, int T, int8_t* mem_k,
                       float* mem_ks, int8_t* mem_v, float* mem_vs) {
    const int d = c->d_model, H = c->heads, hd = c->head_dim;
    float* in = fbuf((size_t)T * d);
    float* kv = fbuf((size_t)T * 2 * d);
    for (size_t i = 0; i < (size_t)T * d; ++i) in[i] = encoded[i] + m->cross_position[i];
    for (int l = 0; l < c->dec_layers; ++l) {
        const ro_wdec_layer* L = &m->dec[l];
        ro_multiply(RO_FORM_PANEL, L->cross_kv.codes, L->cross_kv.scales, 2 * d, d, c->group, in, T, kv, NULL, NULL,
                    NULL);
        size_t base = (size_t)l * T * d, sbase = (size_t)l * T * H;
        for (int t = 0; t < T; ++t) {
            float* row = kv + (size_t)t * 2 * d;
            for (int h = 0; h < H; ++h) {
                size_t o = base + (size_t)t * d + (size_t)h * hd, so = sbase + (size_t)t * H + h;
                mem_ks[so] = head_codes(row + h * hd, hd, L->k_norm, NULL, NULL, mem_k + o);
                mem_vs[so] = head_codes(row + d + h * hd, hd, NULL, NULL, NULL, mem_v + o);
            }
        }
    }
    free(kv);
    free(in);
}

static size_t wcache_offset(const ro_wconfig* c, const ro_wsession* s, int layer, int head, int pos) {
    return (((size_t)layer * c->heads + head) * (size_t)s->capacity + (size_t)pos) * (size_t)c->head_dim;
}

/* CrossState::apply (cross.rs:126-182) without the gate projection: norm,
 * q product, per head q_norm + int8 codes, int8 attention over the memory,
 * out product, post norm, x += gain * attended. */
static void cross_apply(const ro_wconfig* c, const ro_wmodel* m, const ro_wsession* s, int layer, float* x) {
    const ro_wdec_layer* L = &m->dec[layer];
    const int d = c->d_model, H = c->heads, hd = c->head_dim, T = s->frames, g = c->group;
    float normed[4096], q[4096], context[4096], attended[4096], post[4096];
    int8_t qc[4096];
    ro_zero_centred_norm(x, L->norm_cross, d, normed);
    ro_multiply(RO_FORM_PANEL, L->cross_q.codes, L->cross_q.scales, d, d, g, normed, 1, q, NULL, NULL, NULL);
    const float inverse_root = 1.0f / sqrtf((float)hd);
    size_t base = (size_t)layer * T * d, sbase = (size_t)layer * T * H;
    for (int h = 0; h < H; ++h) {
        float qscale = head_codes(q + h * hd, hd, L->q_norm, NULL, NULL, qc + h * hd) * inverse_root;
        ro_int8_attend(qc + h * hd, qscale, s->mem_k + base + h * hd, s->mem_ks + sbase + h, s->mem_v + base + h * hd,
                       s->mem_vs + sbase + h, T, hd, d, H, context + h * hd);
    }
    ro_multiply(RO_FORM_PANEL, L->cross_out.codes, L->cross_out.scales, d, d, g, context, 1, attended, NULL, NULL,
                NULL);
    ro_zero_centred_norm(attended, L->post_norm, d, post);
    for (int i = 0; i < d; ++i) x[i] = x[i] + L->cross_gain * post[i];
}

void ro_whistle_push(const ro_wconfig* c, const ro_wmodel* m, ro_wsession* s, uint32_t token) {
    const int d = c->d_model, H = c->heads, hd = c->head_dim, half = hd / 2, g = c->group;
    const int pos = s->length;
    float* x = fbuf((size_t)d);
    float* normed = fbuf((size_t)d);
    float* qkv = fbuf((size_t)3 * d);
    float* att = fbuf((size_t)d);
    float* y = fbuf((size_t)d);
    {
        const int8_t* row = m->embedding.codes + (size_t)token * d;
        const float* srow = m->embedding.scales + (size_t)token * (d / g);
        float root = sqrtf((float)d);
        for (int k = 0; k < d; ++k) x[k] = ((float)row[k] * srow[k / g]) * root;
    }
    const float* cs = m->rope_cos + (size_t)pos * half;
    const float* sn = m->rope_sin + (size_t)pos * half;
    for (int l = 0; l < c->dec_layers; ++l) {
        const ro_wdec_layer* L = &m->dec[l];
        ro_zero_centred_norm(x, L->norm_attn, d, normed);
        ro_multiply(RO_FORM_PANEL, L->qkv.codes, L->qkv.scales, 3 * d, d, g, normed, 1, qkv, NULL, NULL, NULL);
        for (int h = 0; h < H; ++h) {
            ro_apply_rotary(qkv + h * hd, hd, cs, sn);
            ro_apply_rotary(qkv + d + h * hd, hd, cs, sn);
            size_t off = wcache_offset(c, s, l, h, pos);
            for (int i = 0; i < hd; ++i) {
                s->keys[off + i] = ro_f32_to_f16(qkv[d + h * hd + i]);
                s->values[off + i] = ro_f32_to_f16(qkv[2 * d + h * hd + i]);
            }
            ro_attend_head(qkv + h * hd, s->keys + wcache_offset(c, s, l, h, 0), s->values + wcache_offset(c, s, l, h, 0),
                           hd, pos + 1, att + h * hd);
        }
        ro_multiply(RO_FORM_PANEL, L->out.codes, L->out.scales, d, d, g, att, 1, y, NULL, NULL, NULL);
        for (int i = 0; i < d; ++i) x[i] = x[i] + y[i];
        cross_apply(c, m, s, l, x);
        gated_ffn(c, L->gate_up, L->down, L->norm_ffn, x, 1);
    }
    s->length = pos + 1;
    ro_zero_centred_norm(x, m->dec_norm, d, s->hidden);
    free(y);
    free(att);
    free(qkv);
    free(normed);
    free(x);
}

void ro_whistle_logits(const ro_wconfig* c, const ro_wmodel* m, const ro_wsession* s, float* logits) {
    ro_multiply(RO_FORM_PLANE, m->embedding.codes, m->embedding.scales, c->vocab, c->d_model, c->group, s->hidden, 1,
                logits, NULL, NULL, NULL);
}

void ro_whistle_greedy(const ro_wconfig* c, const ro_wmodel* m, ro_wsession* s, uint32_t first, int steps,
                       uint32_t* ids) {
    float* logits = fbuf((size_t)c->vocab);
    uint32_t token = first;
    for (int step = 0; step < steps; ++step) {
        ro_whistle_push(c, m, s, token);
        ro_whistle_logits(c, m, s, logits);
        token = ro_argmax(logits, c->vocab);
        ids[step] = token;
    }
    free(logits);
}
