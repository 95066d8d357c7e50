/*
 * rn_needle3.c — CPU oracle for the Needle 3 token step (test infrastructure,
 * see rn_oracle.h; never the product path).
 *
 * Restates, function by function:
 *   the archive header, directory and canonical layout (crates/cact/src/
 *     geometry.rs:40-110, archive.rs:43-91, layout.rs:176-257);
 *   ModelConfig (model/src/config.rs), Model::with_depth (model.rs:68-78) and
 *     the head row selection (heads.rs:51-82);
 *   the codebook matrices' dispatch (kernels/src/matrix.rs:155-205): 2-, 4-bit
 *     and ternary matrices the integer path of the reference's aarch64 build,
 *     1- and 3-bit ones the float path;
 *   Session::push and logits (session.rs:76-165), lane_mean and add_engram
 *     (session.rs:175-200);
 *   LaneWeights::route / combine_into / block_delta (lanes.rs:48-104);
 *   table_indices and EngramSiteState::contribute (engram.rs:30-112);
 *   AttentionWeights::attend (model/src/attention.rs:96-154), mix_taps
 *     (:84-94), window_start (:172-178), attend_heads (:180-218);
 *   attend_head as the aarch64 build runs it (kernels/src/attention.rs:53-80
 *     with neon.rs:278-311 softmax_weights and neon.rs:347-438, whose 12-bit
 *     coefficients split into 6-bit halves give the exact integer sum of
 *     round(c / scale) * code);
 *   HadamardWeights::apply (hadamard.rs:55-107) over kronecker_apply's aarch64
 *     32 x 32 path (ops.rs:220-297);
 *   ProbeHead::observe / pooled / project (heads.rs:84-150).
 * f32::exp is the C library's expf, as in the reference.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "rn_oracle.h"

#define N3_HASH_SEED 0x9E3779B9u  /* engram.rs:9-10 */
#define N3_HASH_PRIME 0x01000193u
#define N3_COEFFICIENT_LEVELS 2047.0f /* kernels/src/attention.rs:3 */
#define N3_CHAINS_RANK 8          /* hadamard.rs:6 */
#define N3_HEADER 196

static float* fbuf(size_t n) { return (float*)calloc(n ? n : 1, sizeof(float)); }
static uint32_t rd32(const uint8_t* p) { uint32_t v; memcpy(&v, p, 4); return v; }
static uint64_t rd64(const uint8_t* p) { uint64_t v; memcpy(&v, p, 8); return v; }

/* Iterator::sum of f32 folds from -0.0 */
static float sum_products(const float* a, const float* b, int n) {
    float s = -0.0f;
    for (int i = 0; i < n; ++i) s = s + a[i] * b[i];
    return s;
}

/* ops.rs:19-30: eight strided lanes, the lanes summed in order (from -0.0),
 * then the tail (its own sum from -0.0) */
static float dot_product(const float* a, const float* b, int n) {
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int chunks = n / 8;
    for (int c = 0; c < chunks; ++c)
        for (int j = 0; j < 8; ++j) lanes[j] = lanes[j] + a[8 * c + j] * b[8 * c + j];
    float tail = -0.0f;
    for (int i = chunks * 8; i < n; ++i) tail = tail + a[i] * b[i];
    float total = -0.0f;
    for (int j = 0; j < 8; ++j) total = total + lanes[j];
    return total + tail;
}

static float libm_sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

/* ops.rs:52-58 */
static void norm_in_place(float* v, const float* gain, int n) {
    const float mean_square = ro_sum_of_squares(v, n) / (float)n;
    const float inverse = 1.0f / sqrtf(mean_square + 1e-6f);
    for (int i = 0; i < n; ++i) v[i] = ((1.0f + gain[i]) * v[i]) * inverse;
}

/* session.rs:190-200 */
static void lane_mean(const float* stream, int width, int lanes, float* mean) {
    for (int i = 0; i < width; ++i) mean[i] = 0.0f;
    for (int l = 0; l < lanes; ++l)
        for (int i = 0; i < width; ++i) mean[i] = mean[i] + stream[(size_t)l * width + i] / (float)lanes;
}

/* ---- codebook matrices ---------------------------------------------------- */

void ro_cbm_init(ro_cbm* m, const uint8_t* blob, int rows, int columns, int group, int bits, const float* codebook) {
    const int ib = bits == 5 ? 2 : bits;
    m->rows = rows;
    m->columns = columns;
    m->group = group;
    m->bits = bits;
    m->padded = (columns + group - 1) / group * group;
    m->groups = m->padded / group;
    m->row_bytes = (size_t)m->padded * ib / 8;
    m->packed = blob;
    m->norms = (const uint16_t*)(blob + m->row_bytes * rows);
    const int count = ro_codebook_levels(codebook, bits, group, m->levels);
    m->lscale = ro_integer_levels(m->levels, count, m->table);
    /* integer levels exist for 2-bit, 4-bit and ternary codebooks (matrix.rs:559-
     * 563); groups of 64..256 are multiples of what the panel and plane forms
     * need (matrix.rs:113-121, neon.rs:13-19) */
    m->integer = bits == 2 || bits == 4 || bits == 5;
}

/* QuantisedMatrix::prepare (matrix.rs:123-128) */
void ro_cbm_prepare(const ro_cbm* m, const float* x, float* rotated) {
    ro_codebook_prepare(x, m->columns, m->padded, m->group, rotated);
}

/* fill_rows (matrix.rs:402-421) over rows [first, first + n) for one rotated
 * input: the panel form (2-bit rows starting on a panel of four), the plane
 * form (4-bit, ternary), else fill_rows_float. */
void ro_cbm_rows(const ro_cbm* m, int first, int n, const float* rotated, float* y) {
    const uint8_t* packed = m->packed + (size_t)first * m->row_bytes;
    const uint16_t* norms = m->norms + (size_t)first * m->groups;
    const int integer = m->integer && !(m->bits == 2 && first % 4 != 0);
    if (integer) {
        int8_t* codes = (int8_t*)malloc((size_t)m->padded);
        float* scales = fbuf((size_t)m->groups);
        ro_group_codes(rotated, m->padded, m->group, codes, scales);
        ro_codebook_product(packed, norms, n, m->padded, m->group, m->bits, m->table, m->lscale, codes, scales, 1, y,
                            NULL);
        free(scales);
        free(codes);
    } else {
        ro_codebook_float_vector(packed, norms, n, m->padded, m->group, m->bits, m->levels, rotated, 1, y);
    }
}

/* The product of one token's rotated input as a batched prefill computes it:
 * QuantisedMatrix::multiply_batch (matrix.rs:330-389) takes the integer paths
 * of fill_rows for 2-, 4-bit and ternary matrices, and for the others the float
 * tile (expand_row_scaled, then the eight-lane dot), whose result for a token
 * does not depend on the other tokens of the batch. With batch == 0 this is
 * ro_cbm_rows (multiply_vector / multiply_fused). */
static void cbm_rows_as(const ro_cbm* m, int first, int n, const float* rotated, float* y, int batch) {
    if (batch && !m->integer) {
        ro_codebook_float_batch(m->packed + (size_t)first * m->row_bytes, m->norms + (size_t)first * m->groups, n,
                                m->padded, m->group, m->bits, m->levels, rotated, 1, y);
        return;
    }
    ro_cbm_rows(m, first, n, rotated, y);
}

void ro_cbm_dequantise_row(const ro_cbm* m, int row, float* out) {
    ro_codebook_dequantise_row(m->packed, m->norms, m->padded, m->columns, m->group, m->bits, m->levels, row, out);
}

/* ---- archive and layout ----------------------------------------------------- */

typedef struct {
    int kind, rank;
    uint32_t shape[4];
    uint64_t offset, nbytes;
    uint32_t group, bits;
} n3_record;

typedef struct {
    const uint8_t* bytes;
    size_t size;
    const n3_record* records;
    int count, next, end;
    int failed;
} n3_seq;

static int take(n3_seq* s) {
    if (s->next >= s->end) {
        s->failed = 1;
        return 0;
    }
    return s->next++;
}

/* tensors.rs:3-13 */
static float* floats_of(const n3_seq* s, int index, int* count) {
    const n3_record* r = &s->records[index];
    const uint8_t* p = s->bytes + r->offset;
    int n = 0;
    float* out = NULL;
    if (r->kind == 1) {
        n = (int)(r->nbytes / 2);
        out = fbuf((size_t)n);
        for (int i = 0; i < n; ++i) {
            uint16_t h;
            memcpy(&h, p + 2 * i, 2);
            out[i] = ro_f16_to_f32(h);
        }
    } else if (r->kind == 2) {
        n = (int)(r->nbytes / 4);
        out = fbuf((size_t)n);
        memcpy(out, p, (size_t)n * 4);
    }
    if (count) *count = n;
    return out;
}

static int matrix_of(const n3_seq* s, int index, const float* codebook, ro_cbm* m) {
    const n3_record* r = &s->records[index];
    if (r->kind != 3 || r->rank != 2 || r->bits < 1 || r->bits > 5) return -1;
    if (r->group != 64 && r->group != 128 && r->group != 256) return -1;
    ro_cbm_init(m, s->bytes + r->offset, (int)r->shape[0], (int)r->shape[1], (int)r->group, (int)r->bits, codebook);
    if (m->row_bytes * (size_t)m->rows + (size_t)m->rows * m->groups * 2 > r->nbytes) return -1;
    return 0;
}

static void read_hadamard(n3_seq* s, const float* codebook, int size, ro_n3_hadamard* h) {
    int idx[13];
    for (int i = 0; i < 13; ++i) idx[i] = take(s);
    if (s->failed) return;
    h->size = size;
    h->d1 = floats_of(s, idx[0], NULL);
    h->d2 = floats_of(s, idx[1], NULL);
    h->b2 = floats_of(s, idx[2], NULL);
    h->d3 = floats_of(s, idx[3], NULL);
    h->d4 = floats_of(s, idx[4], NULL);
    for (int f = 0; f < 6; ++f) {
        int n = 0;
        h->factors[f] = floats_of(s, idx[5 + f], &n);
        h->factor_sizes[f] = (int)lround(sqrt((double)n)); /* hadamard.rs:23-25 */
    }
    int nv = 0, nu = 0;
    h->cond_v = floats_of(s, idx[11], &nv);
    h->cond_u = floats_of(s, idx[12], &nu);
    h->rank = nu / size;
    (void)codebook;
    (void)nv;
}

static void free_hadamard(ro_n3_hadamard* h) {
    free(h->d1);
    free(h->d2);
    free(h->b2);
    free(h->d3);
    free(h->d4);
    for (int f = 0; f < 6; ++f) free(h->factors[f]);
    free(h->cond_v);
    free(h->cond_u);
}

/* ladder.rs:1-29 (order by widest-gap bisection, then select the first
 * `depth` of it, sorted); the same rule the product's ladder follows */
static int ladder_select(int layers, int depth, int* out) {
    if (depth == layers) {
        for (int i = 0; i < layers; ++i) out[i] = i;
        return 0;
    }
    if (depth < 2 || depth > layers) return -1;
    int* order = (int*)malloc(sizeof(int) * (size_t)layers);
    int* chosen = (int*)malloc(sizeof(int) * (size_t)layers);
    int n = 0, k = 0;
    order[n++] = 0;
    if (layers > 1) order[n++] = layers - 1;
    while (n < layers) {
        k = 0;
        for (int i = 0; i < n; ++i) chosen[k++] = order[i];
        for (int i = 1; i < k; ++i)
            for (int j = i; j > 0 && chosen[j - 1] > chosen[j]; --j) {
                int t = chosen[j];
                chosen[j] = chosen[j - 1];
                chosen[j - 1] = t;
            }
        int best = -1, best_a = 0, best_b = 0;
        for (int i = 0; i + 1 < k; ++i) {
            const int gap = chosen[i + 1] - chosen[i];
            if (gap > 1 && gap > best) {
                best = gap;
                best_a = chosen[i];
                best_b = chosen[i + 1];
            }
        }
        order[n++] = (best_a + best_b) / 2;
    }
    for (int i = 0; i < depth; ++i) out[i] = order[i];
    for (int i = 1; i < depth; ++i)
        for (int j = i; j > 0 && out[j - 1] > out[j]; --j) {
            int t = out[j];
            out[j] = out[j - 1];
            out[j - 1] = t;
        }
    free(chosen);
    free(order);
    return 0;
}

int ro_n3_open(const uint8_t* bytes, size_t size, int depth, ro_n3_model** out) {
    *out = NULL;
    if (size < N3_HEADER || rd32(bytes) != 0x05E12A84u) return -1;
    if ((size_t)N3_HEADER + 4 * (size_t)rd32(bytes + 8) + 44 * (size_t)rd32(bytes + 4) > size) return -1;
    ro_n3_model* m = (ro_n3_model*)calloc(1, sizeof(ro_n3_model));
    ro_n3_config* c = &m->config;
    const uint8_t* h = bytes + 4;
    uint32_t f[25];
    for (int i = 0; i < 25; ++i) f[i] = rd32(h + 4 * i);
    const int tensor_count = (int)f[0], codebook_len = (int)f[1];
    c->vocab = (int)f[4];
    c->output_vocab = f[5] ? (int)f[5] : (int)f[4]; /* geometry.rs:117-123 */
    c->d_model = (int)f[6];
    c->num_heads = (int)f[7];
    c->num_kv_heads = (int)f[8];
    c->num_layers = (int)f[9];
    c->qk_head_dim = (int)f[10];
    c->v_head_dim = (int)f[11];
    c->max_seq_len = (int)f[12];
    c->hadamard_size = (int)f[13];
    c->lanes = (int)f[14];
    c->sliding_window = (int)f[15];
    c->global_layers = (uint64_t)f[16] | ((uint64_t)f[17] << 32);
    c->conv_taps = (int)f[18];
    c->engram_slots = (int)f[19];
    c->engram_sub_dim = (int)f[20];
    c->engram_tables = (int)f[21];
    c->engram_conv_taps = (int)f[22];
    c->engram_dilation = (int)f[23];
    c->engram_seed_heads = (int)f[24];
    c->engram_order_count = (int)rd32(h + 100);
    for (int i = 0; i < 4; ++i) c->engram_orders[i] = (int)rd32(h + 104 + 4 * i);
    c->engram_site_count = (int)rd32(h + 120);
    for (int i = 0; i < 16; ++i) c->engram_sites[i] = (int)rd32(h + 124 + 4 * i);
    memcpy(&c->rope_theta, h + 188, 4);
    c->engram_heads_per_order = c->engram_tables / (c->engram_order_count > 1 ? c->engram_order_count : 1);
    if (c->engram_order_count > 4 || c->engram_site_count > 16) goto bad;

    memcpy(m->codebook, bytes + N3_HEADER, sizeof(float) * (size_t)(codebook_len < 28 ? codebook_len : 28));
    n3_record* rec = (n3_record*)calloc((size_t)tensor_count, sizeof(n3_record));
    const uint8_t* dir = bytes + N3_HEADER + 4 * (size_t)codebook_len;
    for (int i = 0; i < tensor_count; ++i) {
        const uint8_t* r = dir + 44 * (size_t)i;
        rec[i].kind = r[0];
        rec[i].rank = r[1];
        for (int j = 0; j < 4; ++j) rec[i].shape[j] = rd32(r + 4 + 4 * j);
        rec[i].offset = rd64(r + 20);
        rec[i].nbytes = rd64(r + 28);
        rec[i].group = rd32(r + 36);
        rec[i].bits = rd32(r + 40);
        /* archive.rs:52-66: every tensor inside the file */
        if ((size_t)(dir - bytes) + 44 * (size_t)(i + 1) > size || rec[i].offset > size ||
            rec[i].nbytes > size - rec[i].offset) {
            m->records = rec;
            goto bad;
        }
    }
    m->records = rec;
    if (tensor_count < 1 || rec[tensor_count - 1].kind != 4) goto bad; /* the trailing tokenizer blob */
    n3_seq s = {bytes, size, rec, tensor_count, 0, tensor_count - 1, 0};
    const float* cb = m->codebook;
    const int L = c->num_layers;
    if (matrix_of(&s, take(&s), cb, &m->embedding)) goto bad;
    m->layers = (ro_n3_layer*)calloc((size_t)L, sizeof(ro_n3_layer));
    for (int l = 0; l < L; ++l) {
        ro_n3_layer* y = &m->layers[l];
        y->norm_in = floats_of(&s, take(&s), NULL);
        if (matrix_of(&s, take(&s), cb, &y->q) || matrix_of(&s, take(&s), cb, &y->k) ||
            matrix_of(&s, take(&s), cb, &y->v))
            goto bad;
        if (c->conv_taps > 0)
            for (int t = 0; t < 3; ++t) y->taps[t] = floats_of(&s, take(&s), NULL);
        y->q_norm = floats_of(&s, take(&s), NULL);
        y->k_norm = floats_of(&s, take(&s), NULL);
        if (matrix_of(&s, take(&s), cb, &y->gate) || matrix_of(&s, take(&s), cb, &y->out)) goto bad;
        y->post_norm = floats_of(&s, take(&s), NULL);
        float* g = floats_of(&s, take(&s), NULL);
        y->attention_gate = g ? g[0] : 0.0f;
        free(g);
        y->pre_hadamard_norm = floats_of(&s, take(&s), NULL);
        read_hadamard(&s, cb, c->hadamard_size, &y->hadamard);
        if (s.failed) goto bad;
    }
    /* lanes.rs:31-45 */
    m->a_pre = floats_of(&s, take(&s), NULL);
    m->a_post = floats_of(&s, take(&s), NULL);
    m->a_res = floats_of(&s, take(&s), NULL);
    m->b_pre = floats_of(&s, take(&s), NULL);
    m->b_post = floats_of(&s, take(&s), NULL);
    m->b_res = floats_of(&s, take(&s), NULL);
    if (matrix_of(&s, take(&s), cb, &m->phi_pre) || matrix_of(&s, take(&s), cb, &m->phi_post) ||
        matrix_of(&s, take(&s), cb, &m->phi_res))
        goto bad;
    for (int p = 0; p < 2; ++p) { /* hadamard.rs:36: the permutations as floats, `as usize` */
        int n = 0;
        float* v = floats_of(&s, take(&s), &n);
        m->permutations[p] = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n ? n : 1));
        for (int i = 0; i < n; ++i) m->permutations[p][i] = (int32_t)v[i];
        free(v);
    }
    m->engrams = (ro_n3_engram*)calloc((size_t)(c->engram_site_count ? c->engram_site_count : 1), sizeof(ro_n3_engram));
    for (int e = 0; e < c->engram_site_count; ++e) {
        ro_n3_engram* g = &m->engrams[e];
        if (matrix_of(&s, take(&s), cb, &g->tables) || matrix_of(&s, take(&s), cb, &g->key) ||
            matrix_of(&s, take(&s), cb, &g->value))
            goto bad;
        g->taps = floats_of(&s, take(&s), NULL);
    }
    m->final_norm = floats_of(&s, take(&s), NULL);
    if (s.failed) goto bad;

    /* active layers (model.rs:68-78) */
    if (depth <= 0) depth = L;
    m->active = (int*)malloc(sizeof(int) * (size_t)L);
    if (ladder_select(L, depth, m->active)) {
        ro_n3_close(m);
        return -2;
    }
    m->active_count = depth;

    /* probe heads (layout.rs:228-246, heads.rs:33-82) */
    if (s.next < s.end && rec[s.next].kind == 1) {
        int n = 0;
        float* codes = floats_of(&s, take(&s), &n);
        m->heads = (ro_n3_head*)calloc((size_t)(n ? n : 1), sizeof(ro_n3_head));
        m->head_count = n;
        const int slots_layers = L + 1;
        for (int i = 0; i < n; ++i) {
            ro_n3_head* hd = &m->heads[i];
            hd->code = (int)lroundf(codes[i]);
            if (hd->code < 1 || hd->code > 3) {
                free(codes);
                goto bad;
            }
            ro_cbm probes, query;
            if (matrix_of(&s, take(&s), cb, &probes)) goto bad;
            float* gain = floats_of(&s, take(&s), NULL);
            if (matrix_of(&s, take(&s), cb, &query)) goto bad;
            float* row_bias = floats_of(&s, take(&s), NULL);
            if (matrix_of(&s, take(&s), cb, &hd->projection)) goto bad;
            hd->bias = floats_of(&s, take(&s), NULL);
            if (hd->code == 3) take(&s); /* calibration */
            const int width = probes.columns, k = probes.rows / slots_layers;
            hd->width = width;
            hd->probes_per_layer = k;
            hd->queries = query.rows;
            hd->query = fbuf((size_t)query.rows * width);
            for (int r = 0; r < query.rows; ++r) ro_cbm_dequantise_row(&query, r, hd->query + (size_t)r * width);
            /* with_rows over [0] + active + 1 */
            const int rows = depth + 1;
            hd->layers = rows;
            const int old_slots = slots_layers * k, slots = rows * k;
            hd->probes = fbuf((size_t)slots * width);
            hd->gain = fbuf((size_t)slots);
            hd->row_bias = fbuf((size_t)hd->queries * slots);
            float* dense = fbuf((size_t)width);
            for (int ri = 0; ri < rows; ++ri) {
                const int row = ri == 0 ? 0 : m->active[ri - 1] + 1;
                for (int p = 0; p < k; ++p) {
                    ro_cbm_dequantise_row(&probes, row * k + p, dense);
                    memcpy(hd->probes + ((size_t)ri * k + p) * width, dense, sizeof(float) * (size_t)width);
                    hd->gain[ri * k + p] = gain[row * k + p];
                }
            }
            for (int q = 0; q < hd->queries; ++q)
                for (int ri = 0; ri < rows; ++ri) {
                    const int row = ri == 0 ? 0 : m->active[ri - 1] + 1;
                    for (int p = 0; p < k; ++p)
                        hd->row_bias[(size_t)q * slots + ri * k + p] = row_bias[(size_t)q * old_slots + row * k + p];
                }
            free(dense);
            free(gain);
            free(row_bias);
        }
        free(codes);
    }
    if (s.failed) goto bad;
    if (s.next < s.end) goto bad; /* an audio encoder or left-over tensors: not part of this oracle */
    *out = m;
    return 0;
bad:
    ro_n3_close(m);
    return -1;
}

void ro_n3_close(ro_n3_model* m) {
    if (!m) return;
    const ro_n3_config* c = &m->config;
    if (m->layers) {
        for (int l = 0; l < c->num_layers; ++l) {
            ro_n3_layer* y = &m->layers[l];
            free(y->norm_in);
            for (int t = 0; t < 3; ++t) free(y->taps[t]);
            free(y->q_norm);
            free(y->k_norm);
            free(y->post_norm);
            free(y->pre_hadamard_norm);
            free_hadamard(&y->hadamard);
        }
        free(m->layers);
    }
    free(m->a_pre);
    free(m->a_post);
    free(m->a_res);
    free(m->b_pre);
    free(m->b_post);
    free(m->b_res);
    free(m->permutations[0]);
    free(m->permutations[1]);
    if (m->engrams) {
        for (int e = 0; e < c->engram_site_count; ++e) free(m->engrams[e].taps);
        free(m->engrams);
    }
    free(m->final_norm);
    for (int i = 0; i < m->head_count; ++i) {
        free(m->heads[i].probes);
        free(m->heads[i].gain);
        free(m->heads[i].query);
        free(m->heads[i].row_bias);
        free(m->heads[i].bias);
    }
    free(m->heads);
    free(m->active);
    free(m->records);
    free(m);
}

const ro_n3_config* ro_n3_config_of(const ro_n3_model* m) { return &m->config; }
int ro_n3_active(const ro_n3_model* m, int* layers) {
    if (layers) memcpy(layers, m->active, sizeof(int) * (size_t)m->active_count);
    return m->active_count;
}

/* ---- pieces ----------------------------------------------------------------- */

/* engram.rs:30-46 */
void ro_n3_table_indices(const ro_n3_config* c, const uint32_t* tokens, int position, int* indices) {
    const int stride = c->engram_seed_heads == 0 ? c->engram_heads_per_order : c->engram_seed_heads;
    int n = 0;
    for (int o = 0; o < c->engram_order_count; ++o)
        for (int head = 0; head < c->engram_heads_per_order; ++head) {
            uint32_t acc = N3_HASH_SEED * (uint32_t)(o * stride + head + 1);
            for (int back = 0; back < c->engram_orders[o]; ++back) {
                const uint32_t token = position >= back ? tokens[position - back] : 0u;
                acc = (acc ^ token) * N3_HASH_PRIME;
            }
            acc ^= acc >> 15;
            indices[n++] = (int)(acc % (uint32_t)c->engram_slots);
        }
}

/* hadamard.rs:55-107 */
void ro_n3_hadamard_apply(const ro_n3_hadamard* h, const int32_t* first_perm, const int32_t* second_perm,
                          const float* input, int width, float* output) {
    const int size = h->size, rank = h->rank;
    float* weights = fbuf((size_t)rank);
    if (rank == N3_CHAINS_RANK) {
        float chains[4][N3_CHAINS_RANK];
        memset(chains, 0, sizeof chains);
        for (int g0 = 0; g0 < width; g0 += 4)
            for (int j = 0; j < 4 && g0 + j < width; ++j) {
                const float value = input[g0 + j];
                const float* row = h->cond_v + (size_t)(g0 + j) * N3_CHAINS_RANK;
                for (int r = 0; r < N3_CHAINS_RANK; ++r) chains[j][r] = chains[j][r] + value * row[r];
            }
        for (int j = 0; j < 4; ++j)
            for (int r = 0; r < N3_CHAINS_RANK; ++r) weights[r] = weights[r] + chains[j][r];
    } else {
        for (int d = 0; d < width; ++d)
            for (int r = 0; r < rank; ++r) weights[r] = weights[r] + input[d] * h->cond_v[(size_t)d * rank + r];
    }
    ro_softmax_in_place(weights, rank);
    float* modulation = fbuf((size_t)size);
    for (int i = 0; i < size; ++i) modulation[i] = 1.0f;
    for (int r = 0; r < rank; ++r)
        for (int i = 0; i < size; ++i) modulation[i] = modulation[i] + weights[r] * h->cond_u[(size_t)r * size + i];
    float* scaled = fbuf((size_t)size);
    float* stage = fbuf((size_t)size);
    for (int i = 0; i < size; ++i) scaled[i] = (i < width ? input[i] : 0.0f) * h->d1[i];
    ro_kronecker_apply_32(scaled, h->factors[0], h->factors[1], stage);
    for (int i = 0; i < size; ++i) {
        const float gathered = stage[first_perm[i]];
        scaled[i] = ro_silu(((h->d2[i] * modulation[i]) * gathered) + h->b2[i]);
    }
    ro_kronecker_apply_32(scaled, h->factors[2], h->factors[3], stage);
    for (int i = 0; i < size; ++i) scaled[i] = stage[second_perm[i]] * h->d3[i];
    ro_kronecker_apply_32(scaled, h->factors[4], h->factors[5], stage);
    for (int i = 0; i < width; ++i) output[i] = stage[i] * h->d4[i];
    free(stage);
    free(scaled);
    free(modulation);
    free(weights);
}

/* hadamard.rs:55-107 over explicit arrays: factors [6][32][32] (w1a w1b w2a w2b
 * w3a w3b), cond_v [width][rank], cond_u [rank][size] */
void ro_n3_hadamard_arrays(int size, int rank, const float* d1, const float* d2, const float* b2, const float* d3,
                           const float* d4, const float* factors, const float* cond_v, const float* cond_u,
                           const int32_t* first_perm, const int32_t* second_perm, const float* input, int width,
                           float* output) {
    ro_n3_hadamard h;
    memset(&h, 0, sizeof h);
    h.size = size;
    h.rank = rank;
    h.d1 = (float*)d1;
    h.d2 = (float*)d2;
    h.b2 = (float*)b2;
    h.d3 = (float*)d3;
    h.d4 = (float*)d4;
    for (int f = 0; f < 6; ++f) {
        h.factors[f] = (float*)(factors + (size_t)f * 1024);
        h.factor_sizes[f] = 32;
    }
    h.cond_v = (float*)cond_v;
    h.cond_u = (float*)cond_u;
    ro_n3_hadamard_apply(&h, first_perm, second_perm, input, width, output);
}

/* attend_head (kernels/src/attention.rs:53-80) as its aarch64 build runs it:
 * integer scores; coefficients (score * key_scale) * query_scale; peak;
 * fast_exp of (c - peak) summed in four lanes over the first count - count % 4
 * positions, the lanes added pairwise ((l0 + l1) + (l2 + l3), vaddvq_f32),
 * then the rest in order; c = e * value_scale; the coefficients quantised to
 * round-half-away(c / (peak_c / 2047)) and summed exactly with the value
 * codes (neon.rs:347-438); out = (float)sum * scale, then times 1 / total.
 * keys/values point at the first position, stride between positions. */
void ro_n3_attend_head(const int8_t* query, float query_scale, const int8_t* keys, const float* key_scales,
                       const int8_t* values, const float* value_scales, int count, int qk, int vd, int key_stride,
                       int value_stride, float* out) {
    float* c = fbuf((size_t)count);
    float peak = -INFINITY;
    for (int p = 0; p < count; ++p) {
        int32_t score = 0;
        for (int i = 0; i < qk; ++i) score += (int32_t)query[i] * (int32_t)keys[(size_t)p * key_stride + i];
        c[p] = ((float)score * key_scales[p]) * query_scale;
        peak = fmaxf(peak, c[p]);
    }
    const int vector_count = count - count % 4;
    float lanes[4] = {0, 0, 0, 0};
    for (int p = 0; p < vector_count; ++p) {
        const float e = ro_fast_exp(c[p] - peak);
        lanes[p % 4] = lanes[p % 4] + e;
        c[p] = e * value_scales[p];
    }
    float total = (lanes[0] + lanes[1]) + (lanes[2] + lanes[3]);
    for (int p = vector_count; p < count; ++p) {
        const float e = ro_fast_exp(c[p] - peak);
        total = total + e;
        c[p] = e * value_scales[p];
    }
    const float cpeak = ro_peak_magnitude(c, count);
    if (cpeak <= 0.0f) {
        for (int i = 0; i < vd; ++i) out[i] = 0.0f;
    } else {
        const float scale = cpeak / N3_COEFFICIENT_LEVELS;
        int64_t* sums = (int64_t*)calloc((size_t)vd, sizeof(int64_t));
        for (int p = 0; p < count; ++p) {
            const int32_t w = (int32_t)roundf(c[p] / scale);
            if (w == 0) continue;
            for (int i = 0; i < vd; ++i) sums[i] += (int64_t)w * values[(size_t)p * value_stride + i];
        }
        for (int i = 0; i < vd; ++i) out[i] = (float)(int32_t)sums[i] * scale;
        free(sums);
    }
    const float inverse = 1.0f / total;
    for (int i = 0; i < vd; ++i) out[i] = out[i] * inverse;
    free(c);
}

/* ---- session ---------------------------------------------------------------- */

int ro_n3_session_new(const ro_n3_model* m, int capacity, ro_n3_session** out) {
    const ro_n3_config* c = &m->config;
    ro_n3_session* s = (ro_n3_session*)calloc(1, sizeof(ro_n3_session));
    s->m = m;
    s->capacity = capacity;
    s->tokens = (uint32_t*)calloc((size_t)capacity, sizeof(uint32_t));
    const int L = c->num_layers, qk = c->qk_head_dim, vd = c->v_head_dim, kv = c->num_kv_heads;
    s->caches = (ro_n3_cache*)calloc((size_t)L, sizeof(ro_n3_cache));
    const int qkv = c->num_heads * qk + kv * qk + kv * vd;
    for (int l = 0; l < L; ++l) {
        ro_n3_cache* k = &s->caches[l];
        k->keys = (int8_t*)calloc((size_t)capacity * kv * qk, 1);
        k->values = (int8_t*)calloc((size_t)capacity * kv * vd, 1);
        k->key_scales = fbuf((size_t)capacity * kv);
        k->value_scales = fbuf((size_t)capacity * kv);
        k->history = fbuf((size_t)(c->conv_taps > 0 ? c->conv_taps : 1) * qkv);
    }
    const int keep = (c->engram_conv_taps - 1) * c->engram_dilation + 1;
    s->engram_history = (float**)calloc((size_t)(c->engram_site_count ? c->engram_site_count : 1), sizeof(float*));
    s->engram_count = (int*)calloc((size_t)(c->engram_site_count ? c->engram_site_count : 1), sizeof(int));
    for (int e = 0; e < c->engram_site_count; ++e)
        s->engram_history[e] = fbuf((size_t)(keep > 0 ? keep : 1) * m->engrams[e].value.rows);
    s->cos_tab = fbuf((size_t)capacity * (qk / 2));
    s->sin_tab = fbuf((size_t)capacity * (qk / 2));
    ro_rotary_table(qk, c->rope_theta, capacity, s->cos_tab, s->sin_tab);
    s->hidden = fbuf((size_t)c->d_model);
    s->cells = fbuf((size_t)(m->active_count + 1) * c->d_model);
    s->peak = (float**)calloc((size_t)(m->head_count ? m->head_count : 1), sizeof(float*));
    s->total = (float**)calloc((size_t)(m->head_count ? m->head_count : 1), sizeof(float*));
    s->weighted = (float**)calloc((size_t)(m->head_count ? m->head_count : 1), sizeof(float*));
    for (int i = 0; i < m->head_count; ++i) { /* heads.rs:84-87 */
        const ro_n3_head* h = &m->heads[i];
        const int slots = h->layers * h->probes_per_layer;
        s->peak[i] = fbuf((size_t)slots);
        for (int j = 0; j < slots; ++j) s->peak[i][j] = -INFINITY;
        s->total[i] = fbuf((size_t)slots);
        s->weighted[i] = fbuf((size_t)slots * h->width);
    }
    *out = s;
    return 0;
}

void ro_n3_session_free(ro_n3_session* s) {
    if (!s) return;
    const ro_n3_model* m = s->m;
    const ro_n3_config* c = &m->config;
    for (int l = 0; l < c->num_layers; ++l) {
        free(s->caches[l].keys);
        free(s->caches[l].values);
        free(s->caches[l].key_scales);
        free(s->caches[l].value_scales);
        free(s->caches[l].history);
    }
    free(s->caches);
    for (int e = 0; e < c->engram_site_count; ++e) free(s->engram_history[e]);
    free(s->engram_history);
    free(s->engram_count);
    for (int i = 0; i < m->head_count; ++i) {
        free(s->peak[i]);
        free(s->total[i]);
        free(s->weighted[i]);
    }
    free(s->peak);
    free(s->total);
    free(s->weighted);
    free(s->cos_tab);
    free(s->sin_tab);
    free(s->hidden);
    free(s->cells);
    free(s->tokens);
    free(s);
}

/* #[derive(Clone)] on Session (session.rs:17): every field copied, so the two
 * sessions continue independently (Generator::new/reset, generator.rs:41-46) */
int ro_n3_session_clone(const ro_n3_session* s, ro_n3_session** out) {
    const ro_n3_model* m = s->m;
    const ro_n3_config* c = &m->config;
    ro_n3_session* t = NULL;
    if (ro_n3_session_new(m, s->capacity, &t) != 0) return -1;
    const size_t cap = (size_t)s->capacity;
    const int qk = c->qk_head_dim, vd = c->v_head_dim, kv = c->num_kv_heads;
    const int qkv = c->num_heads * qk + kv * qk + kv * vd;
    t->length = s->length;
    memcpy(t->tokens, s->tokens, cap * sizeof(uint32_t));
    for (int l = 0; l < c->num_layers; ++l) {
        const ro_n3_cache* a = &s->caches[l];
        ro_n3_cache* b = &t->caches[l];
        memcpy(b->keys, a->keys, cap * kv * qk);
        memcpy(b->values, a->values, cap * kv * vd);
        memcpy(b->key_scales, a->key_scales, cap * kv * sizeof(float));
        memcpy(b->value_scales, a->value_scales, cap * kv * sizeof(float));
        memcpy(b->history, a->history, (size_t)(c->conv_taps > 0 ? c->conv_taps : 1) * qkv * sizeof(float));
        b->history_count = a->history_count;
        b->length = a->length;
    }
    const int keep = (c->engram_conv_taps - 1) * c->engram_dilation + 1;
    for (int e = 0; e < c->engram_site_count; ++e) {
        memcpy(t->engram_history[e], s->engram_history[e],
               (size_t)(keep > 0 ? keep : 1) * m->engrams[e].value.rows * sizeof(float));
        t->engram_count[e] = s->engram_count[e];
    }
    memcpy(t->hidden, s->hidden, (size_t)c->d_model * sizeof(float));
    memcpy(t->cells, s->cells, (size_t)(m->active_count + 1) * c->d_model * sizeof(float));
    for (int i = 0; i < m->head_count; ++i) {
        const ro_n3_head* h = &m->heads[i];
        const size_t slots = (size_t)h->layers * h->probes_per_layer;
        memcpy(t->peak[i], s->peak[i], slots * sizeof(float));
        memcpy(t->total[i], s->total[i], slots * sizeof(float));
        memcpy(t->weighted[i], s->weighted[i], slots * h->width * sizeof(float));
    }
    *out = t;
    return 0;
}

/* engram.rs:66-112: contribute for one site */
static void engram_contribute(ro_n3_session* s, int site, const int* indices, int position, float* key, float* value,
                              int batch) {
    const ro_n3_model* m = s->m;
    const ro_n3_config* c = &m->config;
    const ro_n3_engram* g = &m->engrams[site];
    const int sub = c->engram_sub_dim, tables = c->engram_order_count * c->engram_heads_per_order;
    float* gathered = fbuf((size_t)tables * sub);
    float* row = fbuf((size_t)sub);
    for (int t = 0; t < tables; ++t) {
        const int order = c->engram_orders[t / c->engram_heads_per_order];
        if (position + 1 >= order) {
            ro_cbm_dequantise_row(&g->tables, t * c->engram_slots + indices[t], row);
            memcpy(gathered + (size_t)t * sub, row, sizeof(float) * (size_t)sub);
        }
    }
    ro_fake_quantise_int8(gathered, tables * sub);
    float* rotated = fbuf((size_t)g->key.padded);
    ro_cbm_prepare(&g->key, gathered, rotated);
    const int width = g->value.rows;
    float* raw = fbuf((size_t)width);
    cbm_rows_as(&g->key, 0, g->key.rows, rotated, key, batch);    /* engram.rs:84 / contribute_batch :134-136 */
    cbm_rows_as(&g->value, 0, width, rotated, raw, batch);
    const int keep = (c->engram_conv_taps - 1) * c->engram_dilation + 1;
    float* hist = s->engram_history[site];
    memmove(hist + width, hist, sizeof(float) * (size_t)(keep - 1) * width);
    memcpy(hist, raw, sizeof(float) * (size_t)width);
    if (s->engram_count[site] < keep) s->engram_count[site]++;
    for (int i = 0; i < width; ++i) value[i] = 0.0f;
    for (int tap = 0; tap < c->engram_conv_taps; ++tap) {
        const int back = tap * c->engram_dilation;
        if (position < back) continue;
        const float* past = hist + (size_t)back * width;
        const float* gains = g->taps + (size_t)tap * width;
        for (int i = 0; i < width; ++i) value[i] = value[i] + gains[i] * past[i];
    }
    free(raw);
    free(rotated);
    free(row);
    free(gathered);
}

/* session.rs:175-188 */
static void add_engram(float* x, const float* key, const float* value, int width) {
    float* ux = fbuf((size_t)width);
    float* uk = fbuf((size_t)width);
    ro_unit_rms(x, width, ux);
    ro_unit_rms(key, width, uk);
    const float dot = sum_products(ux, uk, width);
    const float alpha = libm_sigmoid(dot / sqrtf((float)width));
    for (int i = 0; i < width; ++i) x[i] = x[i] + alpha * value[i];
    free(uk);
    free(ux);
}

/* attention.rs:84-94 over the history (newest first) of `which` */
static void mix_taps(const float* taps, const float* history, int stride, int offset, int width, int taps_count,
                     int available, int position, float* mixed) {
    for (int i = 0; i < width; ++i) mixed[i] = 0.0f;
    int n = taps_count < position + 1 ? taps_count : position + 1;
    if (n > available) n = available;
    for (int tap = 0; tap < n; ++tap) {
        const float* gains = taps + (size_t)tap * width;
        const float* sample = history + (size_t)tap * stride + offset;
        for (int i = 0; i < width; ++i) mixed[i] = mixed[i] + gains[i] * sample[i];
    }
}

static void apply_rotary_at(const ro_n3_session* s, float* head, int qk, int position) {
    const int half = qk / 2;
    ro_apply_rotary(head, qk, s->cos_tab + (size_t)position * half, s->sin_tab + (size_t)position * half);
}

/* attention.rs:96-154 */
static void attend(ro_n3_session* s, int layer, int position, const float* hidden, float* output, int batch) {
    const ro_n3_model* m = s->m;
    const ro_n3_config* c = &m->config;
    const ro_n3_layer* y = &m->layers[layer];
    ro_n3_cache* cache = &s->caches[layer];
    const int qk = c->qk_head_dim, vd = c->v_head_dim, H = c->num_heads, KV = c->num_kv_heads, d = c->d_model;
    const int qw = H * qk, kw = KV * qk, vw = KV * vd, aw = H * vd, qkv = qw + kw + vw;
    float* quantised = fbuf((size_t)d);
    memcpy(quantised, hidden, sizeof(float) * (size_t)d);
    ro_fake_quantise_int8(quantised, d);
    float* rotated = fbuf((size_t)y->q.padded);
    ro_cbm_prepare(&y->q, quantised, rotated);
    float* q = fbuf((size_t)qw);
    float* k = fbuf((size_t)kw);
    float* v = fbuf((size_t)vw);
    float* gate = fbuf((size_t)aw);
    /* attention.rs:107-110 (multiply_fused) / attend_batch :233-240 (multiply_batch_fused) */
    cbm_rows_as(&y->q, 0, qw, rotated, q, batch);
    cbm_rows_as(&y->k, 0, kw, rotated, k, batch);
    cbm_rows_as(&y->v, 0, vw, rotated, v, batch);
    cbm_rows_as(&y->gate, 0, aw, rotated, gate, batch);
    if (c->conv_taps > 0) {
        float* h = cache->history;
        memmove(h + qkv, h, sizeof(float) * (size_t)(c->conv_taps - 1) * qkv);
        memcpy(h, q, sizeof(float) * (size_t)qw);
        memcpy(h + qw, k, sizeof(float) * (size_t)kw);
        memcpy(h + qw + kw, v, sizeof(float) * (size_t)vw);
        if (cache->history_count < c->conv_taps) cache->history_count++;
        mix_taps(y->taps[0], h, qkv, 0, qw, c->conv_taps, cache->history_count, position, q);
        mix_taps(y->taps[1], h, qkv, qw, kw, c->conv_taps, cache->history_count, position, k);
        mix_taps(y->taps[2], h, qkv, qw + kw, vw, c->conv_taps, cache->history_count, position, v);
    }
    int8_t* qcodes = (int8_t*)malloc((size_t)qw);
    float* qscales = fbuf((size_t)H);
    for (int h = 0; h < H; ++h) {
        float* head = q + (size_t)h * qk;
        norm_in_place(head, y->q_norm, qk);
        apply_rotary_at(s, head, qk, position);
        qscales[h] = ro_quantise_int8(head, qk, qcodes + (size_t)h * qk);
    }
    for (int h = 0; h < KV; ++h) {
        float* head = k + (size_t)h * qk;
        norm_in_place(head, y->k_norm, qk);
        apply_rotary_at(s, head, qk, position);
    }
    for (int h = 0; h < KV; ++h)
        cache->key_scales[(size_t)h * s->capacity + position] =
            ro_quantise_int8(k + (size_t)h * qk, qk, cache->keys + ((size_t)position * KV + h) * qk);
    for (int h = 0; h < KV; ++h)
        cache->value_scales[(size_t)h * s->capacity + position] =
            ro_quantise_int8(v + (size_t)h * vd, vd, cache->values + ((size_t)position * KV + h) * vd);
    cache->length = position + 1;
    /* weighted_values / attend_heads (attention.rs:156-218) */
    const int total = position + 1;
    int first = 0;
    if (c->sliding_window > 0 && !((c->global_layers >> layer) & 1))
        first = total > c->sliding_window ? total - c->sliding_window : 0;
    const int group = H / KV;
    const float inverse_root = 1.0f / sqrtf((float)qk);
    float* attended = fbuf((size_t)aw);
    for (int h = 0; h < H; ++h) {
        const int kvh = h / group;
        ro_n3_attend_head(qcodes + (size_t)h * qk, qscales[h] * inverse_root,
                          cache->keys + ((size_t)first * KV + kvh) * qk, cache->key_scales + (size_t)kvh * s->capacity + first,
                          cache->values + ((size_t)first * KV + kvh) * vd,
                          cache->value_scales + (size_t)kvh * s->capacity + first, total - first, qk, vd, KV * qk,
                          KV * vd, attended + (size_t)h * vd);
    }
    for (int i = 0; i < aw; ++i) attended[i] = attended[i] * libm_sigmoid(gate[i]);
    ro_fake_quantise_int8(attended, aw);
    float* rotated_out = fbuf((size_t)y->out.padded);
    ro_cbm_prepare(&y->out, attended, rotated_out);
    cbm_rows_as(&y->out, 0, y->out.rows, rotated_out, output, batch); /* attention.rs:152 / :359-366 */
    free(rotated_out);
    free(attended);
    free(qscales);
    free(qcodes);
    free(gate);
    free(v);
    free(k);
    free(q);
    free(rotated);
    free(quantised);
}

/* heads.rs:138-155 */
static void heads_observe(ro_n3_session* s) {
    const ro_n3_model* m = s->m;
    for (int i = 0; i < m->head_count; ++i) {
        const ro_n3_head* h = &m->heads[i];
        const int width = h->width, k = h->probes_per_layer;
        const float root = sqrtf((float)width);
        for (int layer = 0; layer < h->layers; ++layer) {
            const float* cell = s->cells + (size_t)layer * width;
            for (int probe = 0; probe < k; ++probe) {
                const int slot = layer * k + probe;
                const float score = dot_product(cell, h->probes + (size_t)slot * width, width) / root;
                const float old = s->peak[i][slot];
                const float peak = fmaxf(old, score);
                const float rescale = old == -INFINITY ? 0.0f : expf(old - peak);
                const float weight = expf(score - peak);
                s->total[i][slot] = s->total[i][slot] * rescale + weight;
                float* target = s->weighted[i] + (size_t)slot * width;
                for (int j = 0; j < width; ++j) target[j] = target[j] * rescale + weight * cell[j];
                s->peak[i][slot] = peak;
            }
        }
    }
}

/* session.rs:76-148 */
/* One token of Session::push (batch == 0) or of Session::prefill (batch == 1):
 * prefill.rs:10-99 runs the same per-token arithmetic as push_with except that
 * the projections and the engram key and value go through multiply_batch. */
static void n3_token(ro_n3_session* s, uint32_t token, int batch) {
    const ro_n3_model* m = s->m;
    const ro_n3_config* c = &m->config;
    const int d = c->d_model, lanes = c->lanes;
    const int position = s->length;
    s->tokens[s->length++] = token;
    float* row = fbuf((size_t)d);
    ro_cbm_dequantise_row(&m->embedding, (int)token, row);
    const float scale = sqrtf((float)d);
    float* stream = fbuf((size_t)lanes * d);
    float* next = fbuf((size_t)lanes * d);
    for (int l = 0; l < lanes; ++l)
        for (int i = 0; i < d; ++i) stream[(size_t)l * d + i] = row[i] * scale;
    lane_mean(stream, d, lanes, s->cells);

    const int tables = c->engram_order_count * c->engram_heads_per_order;
    int* indices = (int*)calloc((size_t)(tables ? tables : 1), sizeof(int));
    ro_n3_table_indices(c, s->tokens, position, indices);
    const int sites = c->engram_site_count;
    float** ekey = (float**)calloc((size_t)(sites ? sites : 1), sizeof(float*));
    float** evalue = (float**)calloc((size_t)(sites ? sites : 1), sizeof(float*));
    for (int e = 0; e < sites; ++e) {
        int present = 0;
        for (int a = 0; a < m->active_count; ++a) present |= m->active[a] == c->engram_sites[e];
        if (!present) continue;
        ekey[e] = fbuf((size_t)m->engrams[e].key.rows);
        evalue[e] = fbuf((size_t)m->engrams[e].value.rows);
        engram_contribute(s, e, indices, position, ekey[e], evalue[e], batch);
    }

    const int phi_padded = m->phi_pre.padded;
    float* normalised = fbuf((size_t)lanes * d);
    float* rotated = fbuf((size_t)phi_padded);
    float* pre = fbuf((size_t)lanes);
    float* post = fbuf((size_t)lanes);
    float* residual = fbuf((size_t)lanes * lanes);
    float* input = fbuf((size_t)d);
    float* x = fbuf((size_t)d);
    float* normed = fbuf((size_t)d);
    float* attended = fbuf((size_t)d);
    float* mlp = fbuf((size_t)d);
    float* delta = fbuf((size_t)d);
    for (int slot = 0; slot < m->active_count; ++slot) {
        const int layer = m->active[slot];
        const ro_n3_layer* y = &m->layers[layer];
        /* lanes.rs:48-84 */
        ro_unit_rms(stream, lanes * d, normalised);
        ro_fake_quantise_int8(normalised, lanes * d);
        ro_cbm_prepare(&m->phi_pre, normalised, rotated);
        ro_cbm_rows(&m->phi_pre, layer * lanes, lanes, rotated, pre);
        ro_cbm_rows(&m->phi_post, layer * lanes, lanes, rotated, post);
        ro_cbm_rows(&m->phi_res, layer * lanes * lanes, lanes * lanes, rotated, residual);
        ro_lanes_route_tail(lanes, d, layer, slot, m->a_pre, m->a_post, m->a_res, m->b_pre, m->b_post, m->b_res,
                            stream, pre, post, residual, input);
        memcpy(x, input, sizeof(float) * (size_t)d);
        for (int e = 0; e < sites; ++e)
            if (c->engram_sites[e] == layer) {
                if (ekey[e]) add_engram(x, ekey[e], evalue[e], d);
                break;
            }
        ro_zero_centred_norm(x, y->norm_in, d, normed);
        attend(s, layer, position, normed, attended, batch);
        norm_in_place(attended, y->post_norm, d);
        const float gate = libm_sigmoid(y->attention_gate);
        for (int i = 0; i < d; ++i) x[i] = x[i] + gate * attended[i];
        ro_zero_centred_norm(x, y->pre_hadamard_norm, d, normed);
        ro_n3_hadamard_apply(&y->hadamard, m->permutations[0], m->permutations[1], normed, d, mlp);
        for (int i = 0; i < d; ++i) x[i] = x[i] + mlp[i];
        for (int i = 0; i < d; ++i) delta[i] = x[i] - input[i];
        ro_lanes_combine(lanes, d, post, residual, stream, delta, next);
        float* t = stream;
        stream = next;
        next = t;
        lane_mean(stream, d, lanes, s->cells + (size_t)(slot + 1) * d);
    }
    float* mean = fbuf((size_t)d);
    lane_mean(stream, d, lanes, mean);
    ro_zero_centred_norm(mean, m->final_norm, d, s->hidden);
    heads_observe(s);
    free(mean);
    free(delta);
    free(mlp);
    free(attended);
    free(normed);
    free(x);
    free(input);
    free(residual);
    free(post);
    free(pre);
    free(rotated);
    free(normalised);
    for (int e = 0; e < sites; ++e) {
        free(ekey[e]);
        free(evalue[e]);
    }
    free(evalue);
    free(ekey);
    free(indices);
    free(next);
    free(stream);
    free(row);
}

/* session.rs:151-165 */
void ro_n3_logits(const ro_n3_session* s, float* logits) {
    const ro_n3_model* m = s->m;
    const int d = m->config.d_model;
    float* q = fbuf((size_t)d);
    memcpy(q, s->hidden, sizeof(float) * (size_t)d);
    ro_fake_quantise_int8(q, d);
    float* rotated = fbuf((size_t)m->embedding.padded);
    ro_cbm_prepare(&m->embedding, q, rotated);
    ro_cbm_rows(&m->embedding, 0, m->config.output_vocab, rotated, logits);
    free(rotated);
    free(q);
}

void ro_n3_push(ro_n3_session* s, uint32_t token) { n3_token(s, token, 0); }

/* Session::feed (session.rs:56-70): at least BATCH_THRESHOLD (4) tokens go in
 * chunks of PREFILL_CHUNK (128), each chunk of at least 4 as a prefill, a
 * shorter last chunk pushed; fewer than 4 tokens are pushed. */
void ro_n3_feed(ro_n3_session* s, const uint32_t* tokens, int count) {
    const int threshold = 4, chunk = 128;
    if (count < threshold) {
        for (int i = 0; i < count; ++i) n3_token(s, tokens[i], 0);
        return;
    }
    for (int i = 0; i < count; i += chunk) {
        const int n = count - i < chunk ? count - i : chunk;
        for (int j = 0; j < n; ++j) n3_token(s, tokens[i + j], n >= threshold);
    }
}

static int head_index(const ro_n3_model* m, int code) {
    for (int i = 0; i < m->head_count; ++i)
        if (m->heads[i].code == code) return i;
    return -1;
}

/* heads.rs:99-125; returns queries * width, or -1 */
int ro_n3_pooled_readout(const ro_n3_session* s, int code, float* pooled) {
    const ro_n3_model* m = s->m;
    const int i = head_index(m, code);
    if (i < 0) return -1;
    const ro_n3_head* h = &m->heads[i];
    const int width = h->width, slots = h->layers * h->probes_per_layer;
    float* readouts = fbuf((size_t)slots * width);
    float* averaged = fbuf((size_t)width);
    for (int slot = 0; slot < slots; ++slot) {
        const float inverse = 1.0f / s->total[i][slot];
        for (int j = 0; j < width; ++j) averaged[j] = s->weighted[i][(size_t)slot * width + j] * inverse;
        float* r = readouts + (size_t)slot * width;
        ro_unit_rms(averaged, width, r);
        for (int j = 0; j < width; ++j) r[j] = r[j] * h->gain[slot];
    }
    const float root = sqrtf((float)width);
    float* weights = fbuf((size_t)slots);
    for (int q = 0; q < h->queries; ++q) {
        const float* query = h->query + (size_t)q * width;
        for (int slot = 0; slot < slots; ++slot)
            weights[slot] = dot_product(readouts + (size_t)slot * width, query, width) / root +
                            h->row_bias[(size_t)q * slots + slot];
        ro_softmax_in_place(weights, slots);
        float* out = pooled + (size_t)q * width;
        for (int j = 0; j < width; ++j) out[j] = 0.0f;
        for (int slot = 0; slot < slots; ++slot)
            for (int j = 0; j < width; ++j) out[j] = out[j] + weights[slot] * readouts[(size_t)slot * width + j];
    }
    free(weights);
    free(averaged);
    free(readouts);
    return h->queries * width;
}

/* heads.rs:127-136 over the pooled readout; returns the projection's rows */
int ro_n3_head_output(const ro_n3_session* s, int code, float* out) {
    const ro_n3_model* m = s->m;
    const int i = head_index(m, code);
    if (i < 0) return -1;
    const ro_n3_head* h = &m->heads[i];
    float* pooled = fbuf((size_t)h->queries * h->width);
    ro_n3_pooled_readout(s, code, pooled);
    float* rotated = fbuf((size_t)h->projection.padded);
    ro_cbm_prepare(&h->projection, pooled, rotated);
    ro_cbm_rows(&h->projection, 0, h->projection.rows, rotated, out);
    for (int r = 0; r < h->projection.rows; ++r) out[r] = out[r] + h->bias[r];
    free(rotated);
    free(pooled);
    return h->projection.rows;
}
