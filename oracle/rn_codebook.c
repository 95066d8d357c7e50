/*
 * rn_codebook.c — CPU oracle for the codebook weight format (test
 * infrastructure, see rn_oracle.h; never the product path).
 *
 * A codebook-quantised [rows][columns] matrix (docs/format.md "Codebook-quantised
 * matrices"; cact record.rs:57-84) pads columns to a multiple of the group size.
 * Its blob holds the packed indices, least-significant bits first
 * (rows x padded x index_bits / 8 bytes), then one fp16 L2 norm per
 * (row, group). Group g of a row is (codebook[idx] * norm) . H with H the
 * normalised Walsh-Hadamard matrix of the group size.
 *
 * The product follows the reference's integer path (the one aarch64 takes):
 *   - the input is rotated group by group (walsh.rs:41-80, matrix.rs:123-128)
 *     and quantised per group to int8 with clamp +-127 (neon.rs:22-106,
 *     panel.rs:52-66);
 *   - the codebook levels become an int8 table with one scale
 *     (IntegerLevels, neon.rs:108-124);
 *   - the exact int32 group sum of table[idx] * code, then per group in order
 *       2-bit (panel.rs:184-188):     total = fmaf(acc, (norm * lscale) * xs, total)
 *       4-bit, ternary (neon.rs:158,180): total = total + (((acc * norm) * lscale) * xs)
 *     (matrix.rs:113-121, 205-214: 2-bit matrices take the panel path, 4-bit
 *     and ternary ones the plane path).
 * 1-bit and 3-bit matrices have no integer path in the reference
 * (matrix.rs:559-563: integer levels for 2 and 4 bits only); they, and every
 * width on x86-64, take the float path, restated by ro_codebook_float_vector
 * (fill_rows_float, matrix.rs:427-440, with LookupTable::dot_group,
 * matrix.rs:610-620) and ro_codebook_float_batch (multiply_batch's float tile,
 * matrix.rs:356-378: expand_row_scaled then the eight-lane dot, matrix.rs:488-497).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "rn_oracle.h"

/* walsh.rs:41-76: radix-2 butterflies with spans 1, 2, 4, ... (the first two
 * fused into the quad stage, which is the same sums), low = a + b, high = a - b,
 * then every value times 1 / sqrt(n) rounded to float. */
void ro_walsh_transform(float* v, int n) {
    int span = 1;
    if (n >= 4) {
        for (int q = 0; q < n; q += 4) {
            const float a = v[q], b = v[q + 1], c = v[q + 2], d = v[q + 3];
            const float low_sum = a + b, low_difference = a - b;
            const float high_sum = c + d, high_difference = c - d;
            v[q] = low_sum + high_sum;
            v[q + 1] = low_difference + high_difference;
            v[q + 2] = low_sum - high_sum;
            v[q + 3] = low_difference - high_difference;
        }
        span = 4;
    }
    for (; span < n; span *= 2)
        for (int block = 0; block < n; block += 2 * span)
            for (int i = block; i < block + span; ++i) {
                const float a = v[i], b = v[i + span];
                v[i] = a + b;
                v[i + span] = a - b;
            }
    const float scale = 1.0f / sqrtf((float)n);
    for (int i = 0; i < n; ++i) v[i] = v[i] * scale;
}

/* matrix.rs:123-138 and walsh.rs:78-80: copy `columns` values, zero-pad to
 * `padded`, rotate each group. */
void ro_codebook_prepare(const float* x, int columns, int padded, int group, float* rotated) {
    memcpy(rotated, x, (size_t)columns * sizeof(float));
    for (int i = columns; i < padded; ++i) rotated[i] = 0.0f;
    for (int g = 0; g < padded; g += group) ro_walsh_transform(rotated + g, group);
}

/* codebook.rs:12-43 and matrix.rs:499-508: the float levels of a bit width,
 * padded with zeros to 16. Returns the count of levels (2^index_bits), 0 for an
 * unknown width. */
int ro_codebook_levels(const float* codebook, int bits, int group, float levels[16]) {
    for (int i = 0; i < 16; ++i) levels[i] = 0.0f;
    switch (bits) {
        case 1: {
            const float level = sqrtf(2.0f / 3.14159265358979323846f) / sqrtf((float)group);
            levels[0] = -level;
            levels[1] = level;
            return 2;
        }
        case 2: memcpy(levels, codebook, 4 * sizeof(float)); return 4;
        case 3: memcpy(levels, codebook + 4, 8 * sizeof(float)); return 8;
        case 4: memcpy(levels, codebook + 12, 16 * sizeof(float)); return 16;
        case 5: {
            const float level = 1.2240064f / sqrtf((float)group);
            levels[1] = level;
            levels[3] = -level;
            return 4;
        }
        default: return 0;
    }
}

/* neon.rs:114-124: scale = peak / 127 (1.0 for a zero peak), table entry =
 * level / scale rounded half away from zero (Rust f32::round). */
float ro_integer_levels(const float levels[16], int count, int8_t table[16]) {
    float peak = 0.0f;
    for (int i = 0; i < count; ++i) peak = fmaxf(peak, fabsf(levels[i]));
    const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    for (int i = 0; i < 16; ++i) table[i] = 0;
    for (int i = 0; i < count; ++i) table[i] = (int8_t)roundf(levels[i] / scale);
    return scale;
}

/* panel.rs:52-66 / neon.rs:63-106: per group, scale = peak / 127 (1.0 for a
 * zero peak) and code = round-half-even(x / scale) clamped to +-127, NaN -> 0.
 * codes in natural order. */
void ro_group_codes(const float* rotated, int n, int group, int8_t* codes, float* scales) {
    for (int g = 0; g < n / group; ++g) {
        const float* s = rotated + (size_t)g * group;
        const float peak = ro_peak_magnitude(s, group);
        const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
        scales[g] = scale;
        for (int i = 0; i < group; ++i) {
            float q = rintf(s[i] / scale);
            q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
            codes[(size_t)g * group + i] = q != q ? 0 : (int8_t)q;
        }
    }
}

static float level_at(const uint8_t* row, int e, int ib, const float levels[16]);

/* record.rs:66-72: the index width in the blob (ternary crumbs are 2 bits) */
static int index_bits(int bits) { return bits == 5 ? 2 : bits; }

/* matrix.rs:623-631: the index of element e of a packed row (LSB first) */
static int code_at(const uint8_t* row, int e, int ib) {
    const int bit = e * ib;
    return (row[bit / 8] >> (bit % 8)) & ((1 << ib) - 1);
}

/* y[t][rows] for `count` inputs given as per-group codes [t][padded] and scales
 * [t][padded/group]; acc (nullable) [t][rows][padded/group]. */
void ro_codebook_product(const uint8_t* packed, const uint16_t* norms, int rows, int padded, int group,
                         int bits, const int8_t table[16], float lscale, const int8_t* xcodes,
                         const float* xscales, int count, float* y, int32_t* acc) {
    const int ib = index_bits(bits), groups = padded / group;
    const size_t row_bytes = (size_t)padded * ib / 8;
#pragma omp parallel for schedule(static) num_threads(ro_get_threads()) if ((size_t)rows * padded * count >= (1u << 18))
    for (int r = 0; r < rows; ++r) {
        const uint8_t* row = packed + (size_t)r * row_bytes;
        for (int t = 0; t < count; ++t) {
            const int8_t* xc = xcodes + (size_t)t * padded;
            const float* xs = xscales + (size_t)t * groups;
            float total = 0.0f;
            for (int g = 0; g < groups; ++g) {
                int32_t a = 0;
                for (int i = 0; i < group; ++i) {
                    const int e = g * group + i;
                    a += (int32_t)table[code_at(row, e, ib)] * (int32_t)xc[e];
                }
                if (acc) acc[((size_t)t * rows + r) * groups + g] = a;
                const float norm = ro_f16_to_f32(norms[(size_t)r * groups + g]);
                if (bits == 2)
                    total = fmaf((float)a, (norm * lscale) * xs[g], total);
                else
                    total = total + ((((float)a * norm) * lscale) * xs[g]);
            }
            y[(size_t)t * rows + r] = total;
        }
    }
}

/* matrix.rs:140-153: out[columns] = per group (level[idx] * norm) then the
 * Walsh-Hadamard transform of the group, truncated to `columns`. */
void ro_codebook_dequantise_row(const uint8_t* packed, const uint16_t* norms, int padded, int columns,
                                int group, int bits, const float levels[16], int row, float* out) {
    const int ib = index_bits(bits), groups = padded / group;
    const uint8_t* r = packed + (size_t)row * padded * ib / 8;
    float* full = (float*)malloc((size_t)padded * sizeof(float));
    for (int g = 0; g < groups; ++g) {
        const float norm = ro_f16_to_f32(norms[(size_t)row * groups + g]);
        for (int i = 0; i < group; ++i) full[g * group + i] = level_at(r, g * group + i, ib, levels) * norm;
        ro_walsh_transform(full + g * group, group);
    }
    memcpy(out, full, (size_t)columns * sizeof(float));
    free(full);
}

/* matrix.rs:623-631: the level of element e of a packed row, LSB first; a
 * 3-bit index may straddle two bytes */
static float level_at(const uint8_t* row, int e, int ib, const float levels[16]) {
    const int bit = e * ib, byte = bit / 8, shift = bit % 8;
    uint32_t raw = row[byte];
    if (shift + ib > 8) raw |= (uint32_t)row[byte + 1] << 8;
    return levels[(raw >> shift) & ((1u << ib) - 1)];
}

/* LookupTable::dot_group (matrix.rs:610-620). 1-, 2- and 4-bit indices (and
 * ternary crumbs) go through per-byte tables: lane l of the 8 / index_bits
 * values of a byte sums entry * input over the group's bytes in order from
 * 0.0 (dot_with, matrix.rs:540-549), then the lanes are summed in order;
 * 3-bit indices sum value * input over the group's positions in order
 * (Bitwise). Iterator::sum of f32 folds from -0.0 (Rust 1.87). */
static float dot_group(const uint8_t* row, int g, int group, int ib, const float levels[16], const float* x) {
    if (ib == 3) {
        float s = -0.0f;
        for (int p = 0; p < group; ++p) s = s + level_at(row, g * group + p, ib, levels) * x[p];
        return s;
    }
    const int n = 8 / ib;
    float lanes[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = 0; b < group / n; ++b)
        for (int l = 0; l < n; ++l) lanes[l] = lanes[l] + level_at(row, g * group + b * n + l, ib, levels) * x[b * n + l];
    float s = -0.0f;
    for (int l = 0; l < n; ++l) s = s + lanes[l];
    return s;
}

/* fill_rows_float (matrix.rs:427-440) for `count` rotated inputs [t][padded]:
 * per row, total = 0, then total += dot_group * norm over the groups in order. */
void ro_codebook_float_vector(const uint8_t* packed, const uint16_t* norms, int rows, int padded, int group, int bits,
                              const float levels[16], const float* rotated, int count, float* y) {
    const int ib = index_bits(bits), groups = padded / group;
    const size_t row_bytes = (size_t)padded * ib / 8;
#pragma omp parallel for schedule(static) num_threads(ro_get_threads()) if ((size_t)rows * padded * count >= (1u << 18))
    for (int r = 0; r < rows; ++r) {
        const uint8_t* row = packed + (size_t)r * row_bytes;
        for (int t = 0; t < count; ++t) {
            const float* x = rotated + (size_t)t * padded;
            float total = 0.0f;
            for (int g = 0; g < groups; ++g)
                total = total + dot_group(row, g, group, ib, levels, x + (size_t)g * group) *
                                    ro_f16_to_f32(norms[(size_t)r * groups + g]);
            y[(size_t)t * rows + r] = total;
        }
    }
}

/* multiply_batch's float tile (matrix.rs:356-378): the row expanded and scaled
 * (expand_row_scaled, matrix.rs:390-399: level * norm per element), then
 * dot (matrix.rs:488-497): eight lanes over chunks of 8 from 0.0, the lanes
 * summed in order from -0.0. */
void ro_codebook_float_batch(const uint8_t* packed, const uint16_t* norms, int rows, int padded, int group, int bits,
                             const float levels[16], const float* rotated, int count, float* y) {
    const int ib = index_bits(bits), groups = padded / group;
    const size_t row_bytes = (size_t)padded * ib / 8;
#pragma omp parallel for schedule(static) num_threads(ro_get_threads()) if ((size_t)rows * padded * count >= (1u << 18))
    for (int r = 0; r < rows; ++r) {
        const uint8_t* row = packed + (size_t)r * row_bytes;
        float* w = (float*)malloc((size_t)padded * sizeof(float));
        for (int e = 0; e < padded; ++e)
            w[e] = level_at(row, e, ib, levels) * ro_f16_to_f32(norms[(size_t)r * groups + e / group]);
        for (int t = 0; t < count; ++t) {
            const float* x = rotated + (size_t)t * padded;
            float lanes[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            for (int c = 0; c < padded / 8; ++c)
                for (int l = 0; l < 8; ++l) lanes[l] = lanes[l] + w[8 * c + l] * x[8 * c + l];
            float s = -0.0f;
            for (int l = 0; l < 8; ++l) s = s + lanes[l];
            y[(size_t)t * rows + r] = s;
        }
        free(w);
    }
}
